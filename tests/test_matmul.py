"""Prefill projections: Q8_0 activation quantizer and the Q1_0 x Q8_0 matmul
(src/forward.rs:415-472, quantize_q8_0.wgsl, matmul_q1_0_q8_0.wgsl).

CPU part: the oracle's layout and arithmetic against closed forms and an f64
brute force. GPU part: the HIP kernels through the C ABI against the oracle,
bit for bit (both follow the reference's f32 operation order exactly; the
integer sums are exact).
"""
import sys

import numpy as np
import pytest

import oracle as orc

HIDDEN, Q_DIM, KV_DIM, FFN = 2560, 4096, 1024, 9728


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


def _q8_layout(m, k):
    """The reference's activation buffer: d region first, qs after it."""
    nb = k // 32
    d_off, qs_off = 0, m * nb * 4
    return d_off, qs_off, qs_off + m * k


def _weights(rng, n, k, pad=256):
    buf, d0, q0 = orc.q1_0_tensor(rng, n, k)
    out = rng.integers(0, 256, pad + buf.size + pad, dtype=np.uint8)
    out[pad:pad + buf.size] = buf
    return out, pad + d0, pad + q0


def _signs(buf, d_off, qs_off, n, k):
    nb = k // 128
    d = buf[d_off:d_off + 2 * n * nb].view(np.float16).astype(np.float64).reshape(n, nb)
    qs = buf[qs_off:qs_off + 16 * n * nb].reshape(n, nb, 16)
    bits = np.unpackbits(qs, axis=-1, bitorder="little").reshape(n, k).astype(np.int64)
    return d, 2 * bits - 1


def _acts(q8, m, k, d_off, qs_off):
    nb = k // 32
    ad = q8[d_off:d_off + 4 * m * nb].view(np.float32).astype(np.float64).reshape(m, nb)
    q = q8[qs_off:qs_off + m * k].view(np.int8).astype(np.int64).reshape(m, k)
    return ad, q


def _brute(wbuf, w_d, w_qs, n, k, q8, m, a_d, a_qs):
    """f64 y[m, n] and the sum of |terms| (for rounding bounds)."""
    wd, s = _signs(wbuf, w_d, w_qs, n, k)
    ad, q = _acts(q8, m, k, a_d, a_qs)
    sumi = np.einsum("mbe,nbe->mnb", q.reshape(m, k // 32, 32), s.reshape(n, k // 32, 32))
    scale = ad[:, None, :] * np.repeat(wd, 4, axis=1)[None, :, :]
    terms = scale * sumi
    return terms.sum(-1), np.abs(terms).sum(-1)


# ---------------------------------------------------------------- CPU: oracle pins
def test_oracle_quantize_layout_and_values():
    """Blocks built as t * c with integer t (|t| <= 127, one of them 127): d = c,
    q = t exactly; d's and qs land at the reference's offsets; nothing else written."""
    rng = np.random.default_rng(0)
    m, k = 5, 96
    nb = k // 32
    t = rng.integers(-127, 128, (m, nb, 32))
    t[:, :, 0] = 127
    c = 2.0 ** rng.integers(-8, 2, (m, nb, 1))
    x = (t * c).astype(np.float16)            # exact in f16
    x[2, 1] = 0                               # all-zero block: d = 0, q = 0
    act = np.concatenate([np.zeros(16, np.uint16), _f16(x.reshape(-1))])
    d_off, qs_off, size = _q8_layout(m, k)
    garbage = rng.integers(0, 256, size + 64, dtype=np.uint8)
    p = orc.QuantParams(k=k, m=m, input_offset=16, d_offset=d_off, qs_offset=qs_off)
    out = orc.quantize_act_q8_0(p, act, garbage)
    ad, q = _acts(out, m, k, d_off, qs_off)
    want_d = (127 * c[..., 0]).astype(np.float32) / np.float32(127)
    want_d[2, 1] = 0
    assert np.array_equal(ad, want_d.astype(np.float64))
    want_q = t.copy()
    want_q[2, 1] = 0
    assert np.array_equal(q.reshape(m, nb, 32), want_q)
    assert np.array_equal(out[size:], garbage[size:])


def test_oracle_quantize_rounds_half_to_even():
    k, m = 32, 1
    # amax 127 -> d = 1: values at .5 round to even
    x = np.zeros(32, np.float32)
    x[0] = 127
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    act = _f16(x)
    d_off, qs_off, size = _q8_layout(m, k)
    out = orc.quantize_act_q8_0(orc.QuantParams(k=k, m=m, input_offset=0, d_offset=d_off, qs_offset=qs_off),
                                act, np.zeros(size, np.uint8))
    _, q = _acts(out, m, k, d_off, qs_off)
    assert list(q[0, :9]) == [127, 0, 2, 2, 0, -2, -2, 126, -126]


def test_oracle_matmul_exact_and_random():
    rng = np.random.default_rng(1)
    m, n, k = 9, 20, 512
    wbuf, w_d, w_qs = _weights(rng, n, k)
    nb1 = k // 128
    # exact case: power-of-two scales, small q -> every f32 op exact
    wbuf[w_d:w_d + 2 * n * nb1] = (2.0 ** rng.integers(-3, 3, n * nb1)).astype(np.float16).view(np.uint8)
    d_off, qs_off, size = _q8_layout(m, k)
    q8 = np.zeros(size, np.uint8)
    q8[d_off:d_off + 4 * m * k // 32] = (2.0 ** rng.integers(-4, 1, m * k // 32)).astype(np.float32).view(np.uint8)
    q8[qs_off:] = rng.integers(-3, 4, m * k).astype(np.int8).view(np.uint8)
    out_off = 32
    y0 = _f16(rng.standard_normal(out_off + m * n))
    p = orc.MatmulParams(k=k, n=n, m=m, w_d_offset=w_d, w_qs_offset=w_qs, a_d_offset=d_off, a_qs_offset=qs_off,
                         out_offset=out_off, accumulate=0)
    y = orc.matmul_q1_0_q8_0(p, wbuf, q8, y0)
    want, _ = _brute(wbuf, w_d, w_qs, n, k, q8, m, d_off, qs_off)
    got = y[out_off:].view(np.float16).astype(np.float64).reshape(m, n)
    assert np.array_equal(got, want.astype(np.float16).astype(np.float64))
    assert np.array_equal(y[:out_off], y0[:out_off])
    # accumulate: f16(f32(y) + acc), exact here too
    p.accumulate = 1
    y2 = orc.matmul_q1_0_q8_0(p, wbuf, q8, y0)
    old = y0[out_off:].view(np.float16).astype(np.float64).reshape(m, n)
    got2 = y2[out_off:].view(np.float16).astype(np.float64).reshape(m, n)
    assert np.array_equal(got2, (old.astype(np.float32) + want.astype(np.float32)).astype(np.float16))
    # random scales: within f32 rounding of the f64 sum, then the f16 store
    wbuf2, w_d2, w_qs2 = _weights(rng, n, k)
    q8r = q8.copy()
    q8r[d_off:d_off + 4 * m * k // 32] = (np.abs(rng.standard_normal(m * k // 32)) * 0.02).astype(np.float32).view(np.uint8)
    q8r[qs_off:] = rng.integers(-127, 128, m * k).astype(np.int8).view(np.uint8)
    p2 = orc.MatmulParams(k=k, n=n, m=m, w_d_offset=w_d2, w_qs_offset=w_qs2, a_d_offset=d_off, a_qs_offset=qs_off,
                          out_offset=out_off, accumulate=0)
    y3 = orc.matmul_q1_0_q8_0(p2, wbuf2, q8r, y0)
    want3, mag = _brute(wbuf2, w_d2, w_qs2, n, k, q8r, m, d_off, qs_off)
    got3 = y3[out_off:].view(np.float16).astype(np.float64).reshape(m, n)
    err = np.abs(got3 - want3)
    tol = 4 * (k // 32) * 2.0**-24 * mag + 2.0**-11 * np.abs(want3) + 2.0**-24
    assert np.all(err <= tol)
    # a sign flip of one element of one weight row would be visible
    assert np.median(np.abs(np.diff(want3, axis=1))) > 100 * np.median(tol)


# ---------------------------------------------------------------- GPU: HIP vs oracle
def _dev(arr):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int8 if arr.dtype == np.uint8 else np.int16)).cuda()


def _host(t, dtype):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype)


def _model():
    import torch
    from bonsai_pot_amd import Model, layout
    m = Model(layout.Config(n_layer=1), 64)
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    return m


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,in_off,shift", [(1, 32, 24, 0), (7, 2560, 24, 0), (64, 4096, 24, 0), (512, 2560, 24, 0),
                                              (100, 9728, 24, 0), (33, 2560, 5, 4), (9, 4096, 2, 8)])
def test_quantize_bit_exact(cuda, m, k, in_off, shift):
    _say(f"[quantize] m={m} k={k} in_off={in_off} shift={shift}")
    rng = np.random.default_rng(m * 7 + k)
    x = (rng.standard_normal(m * k) * np.exp(rng.standard_normal(m * k))).astype(np.float16)
    x[: min(64, x.size)] = 0                      # zero blocks
    act = np.concatenate([_f16(rng.standard_normal(in_off)), _f16(x)])
    d_off, qs_off, size = _q8_layout(m, k)
    d_off, qs_off, size = d_off + shift, qs_off + shift, size + shift   # unaligned to 16 bytes
    q8 = rng.integers(0, 256, size + 256, dtype=np.uint8)
    want = orc.quantize_act_q8_0(orc.QuantParams(k=k, m=m, input_offset=in_off, d_offset=d_off, qs_offset=qs_off),
                                 act, q8)
    a_d, q_d = _dev(act), _dev(q8)
    _model().dispatch_quantize_act(a_d.data_ptr(), q_d.data_ptr(), k, m, in_off, d_off, qs_off)
    got = _host(q_d, np.uint8)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}"


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,acc", [(1, 64, 128, 0), (7, 100, 2560, 1), (64, Q_DIM + 2 * KV_DIM, HIDDEN, 0),
                                       (130, HIDDEN, Q_DIM, 1), (64, 2 * FFN, HIDDEN, 0), (33, HIDDEN, FFN, 1),
                                       (512, 256, HIDDEN, 0)])
def test_matmul_bit_exact(cuda, m, n, k, acc):
    _say(f"[matmul] m={m} n={n} k={k} acc={acc}")
    rng = np.random.default_rng(m + n + k)
    wbuf, w_d, w_qs = _weights(rng, n, k)
    # activations through the oracle quantizer (the reference's pipeline)
    x = rng.standard_normal(m * k).astype(np.float16)
    d_off, qs_off, size = _q8_layout(m, k)
    q8 = orc.quantize_act_q8_0(orc.QuantParams(k=k, m=m, input_offset=0, d_offset=d_off, qs_offset=qs_off),
                               _f16(x), np.zeros(size, np.uint8))
    out_off = 40
    y0 = _f16(rng.standard_normal(out_off + m * n + 40))
    p = orc.MatmulParams(k=k, n=n, m=m, w_d_offset=w_d, w_qs_offset=w_qs, a_d_offset=d_off, a_qs_offset=qs_off,
                         out_offset=out_off, accumulate=acc)
    want = orc.matmul_q1_0_q8_0(p, wbuf, q8, y0)
    w_dv, q_dv, y_dv = _dev(wbuf), _dev(q8), _dev(y0)
    _model().dispatch_matmul_q1_0(w_dv.data_ptr(), q_dv.data_ptr(), y_dv.data_ptr(), k, n, m, w_d, w_qs, d_off,
                                  qs_off, out_off, bool(acc))
    got = _host(y_dv, np.uint16)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} outputs differ, first at {bad[:8]}"


@pytest.mark.gpu
def test_quantize_then_matmul_on_device(cuda):
    """The reference's two-dispatch sequence on the device (quantize into the
    activation buffer, then the matmul reading it) against the oracle's."""
    m, n, k = 96, 512, HIDDEN
    rng = np.random.default_rng(11)
    wbuf, w_d, w_qs = _weights(rng, n, k)
    x = rng.standard_normal(m * k).astype(np.float16)
    act = np.concatenate([_f16(x), np.zeros(m * n, np.uint16)])
    d_off, qs_off, size = _q8_layout(m, k)
    pq = orc.QuantParams(k=k, m=m, input_offset=0, d_offset=d_off, qs_offset=qs_off)
    q8 = orc.quantize_act_q8_0(pq, act, np.zeros(size, np.uint8))
    pm = orc.MatmulParams(k=k, n=n, m=m, w_d_offset=w_d, w_qs_offset=w_qs, a_d_offset=d_off, a_qs_offset=qs_off,
                          out_offset=m * k, accumulate=0)
    want = orc.matmul_q1_0_q8_0(pm, wbuf, q8, act)
    mdl = _model()
    w_dv, a_dv = _dev(wbuf), _dev(act)
    import torch
    q_dv = torch.zeros(size, dtype=torch.int8, device="cuda")
    mdl.dispatch_quantize_act(a_dv.data_ptr(), q_dv.data_ptr(), k, m, 0, d_off, qs_off)
    mdl.dispatch_matmul_q1_0(w_dv.data_ptr(), q_dv.data_ptr(), a_dv.data_ptr(), k, n, m, w_d, w_qs, d_off, qs_off,
                             m * k, False)
    assert np.array_equal(_host(a_dv, np.uint16), want)


@pytest.mark.gpu
def test_matmul_rejects_bad_args(cuda):
    from bonsai_pot_amd.errors import PotError
    import torch
    mdl = _model()
    b = torch.zeros(1 << 16, dtype=torch.int8, device="cuda")
    with pytest.raises(PotError):
        mdl.dispatch_matmul_q1_0(b.data_ptr(), b.data_ptr(), b.data_ptr(), 96, 16, 16, 0, 0, 0, 0, 0, False)
    with pytest.raises(PotError):
        mdl.dispatch_matmul_q1_0(b.data_ptr(), b.data_ptr(), b.data_ptr(), 128, 16, 16, 1, 0, 0, 0, 0, False)
    with pytest.raises(PotError):
        mdl.dispatch_quantize_act(b.data_ptr(), b.data_ptr(), 48, 4, 0, 0, 0)
