"""Top-k of the logits (src/shaders/topk_reduce.wgsl, src/forward.rs:336-354,
:542-568).

CPU part: the oracle's restatement against what does not depend on the
network's tie handling: for distinct logits the result is the sorted top-k
(np.argsort), with the -1e30 / index-0 fill when fewer than k logits exceed
-1e30; with ties the values are still the sorted top-k multiset and every
index names a logit of that value, each index once. Which of several equal
logits is returned (and in which order) is fixed only by the reference's
network; tests/test_topk_wgsl_sim.py pins the oracle's restatement of it
against a second, separately written workgroup simulation of the shader on
tie-heavy inputs.

GPU part: the HIP kernels through the C ABI against the oracle, values and
indices identical, ties included.
"""
import sys

import numpy as np
import pytest

import oracle as orc

VOCAB = 151936


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run_oracle(x16, k, in_off=0, out_off=0, n=None):
    n = x16.size - in_off if n is None else n
    res = np.zeros(out_off + 64 + 8, np.uint32)
    out = orc.topk_reduce(orc.TopKParams(n=n, in_offset=in_off, out_offset=out_off, k=k), x16, res)
    kk = min(k, 32)
    return out[out_off:out_off + kk].view(np.float32), out[out_off + kk:out_off + 2 * kk], out


def _distinct_f16(rng, n):
    """n distinct finite f16 values in random order."""
    pool = np.arange(0x0000, 0x7BFF, dtype=np.uint16)               # +0 .. 65504 (positive finite)
    neg = pool[1:] | np.uint16(0x8000)
    allv = np.concatenate([pool, neg])
    return rng.permutation(allv)[:n].view(np.float16)


@pytest.mark.parametrize("n,k", [(VOCAB, 1), (VOCAB, 8), (VOCAB, 32), (5000, 40), (513, 32), (33, 32), (7, 5)])
def test_oracle_distinct_is_sorted_topk(n, k):
    rng = np.random.default_rng(n + k)
    x = _distinct_f16(rng, n)
    vals, idx, _ = _run_oracle(x.view(np.uint16), k)
    kk = min(k, 32)
    order = np.argsort(-x.astype(np.float64), kind="stable")
    m = min(kk, n)
    assert np.array_equal(idx[:m], order[:m])
    assert np.array_equal(vals[:m], x[order[:m]].astype(np.float32))
    assert np.all(vals[m:] == np.float32(-1e30)) and np.all(idx[m:] == 0)


def test_oracle_ties_keep_value_multiset():
    rng = np.random.default_rng(5)
    x = rng.integers(-20, 12, VOCAB).astype(np.float16)               # heavy ties
    vals, idx, _ = _run_oracle(x.view(np.uint16), 32)
    want = np.sort(x.astype(np.float32))[::-1][:32]
    assert np.array_equal(vals, want)
    assert np.unique(idx).size == 32
    assert np.array_equal(x[idx].astype(np.float32), vals)


def test_oracle_special_values_and_fill():
    x = np.full(100, -np.inf, np.float16)
    x[[3, 50]] = np.nan
    x[7] = np.inf
    x[9] = -65504.0
    vals, idx, _ = _run_oracle(x.view(np.uint16), 4)
    # NaN and -inf never pass the strict `v > min` test; +inf does
    assert vals[0] == np.inf and idx[0] == 7
    assert vals[1] == np.float32(-65504.0) and idx[1] == 9
    assert np.all(vals[2:] == np.float32(-1e30)) and np.all(idx[2:] == 0)
    vals, idx, _ = _run_oracle(np.zeros(0, np.uint16), 3, n=0)
    assert np.all(vals == np.float32(-1e30)) and np.all(idx == 0)


def test_oracle_offsets_and_odd_tail():
    rng = np.random.default_rng(9)
    x = _distinct_f16(rng, 1001)
    buf = np.concatenate([np.full(6, 60000.0, np.float16), x, np.full(3, 65000.0, np.float16)])
    # in_offset 6 (even), n = 1001 (odd): the word holding element 1000 also holds
    # the first trailing 65000, which the n bound must exclude
    vals, idx, out = _run_oracle(buf.view(np.uint16), 16, in_off=6, out_off=5, n=1001)
    order = np.argsort(-x.astype(np.float64))[:16]
    assert np.array_equal(idx, order) and np.array_equal(vals, x[order].astype(np.float32))
    assert np.all(out[:5] == 0)


# ---------------------------------------------------------------- GPU: HIP vs oracle
def _model():
    import torch
    from bonsai_pot_amd import Model, layout
    m = Model(layout.Config(n_layer=1), 64)
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    return m


def _gpu(m, x16, k, in_off, out_off, n):
    import torch
    # two spare elements: an odd n reads the word that holds element n as well
    padded = np.concatenate([np.ascontiguousarray(x16), np.zeros(2, np.uint16)])
    act = torch.from_numpy(padded.view(np.int16)).cuda()
    res = torch.zeros(out_off + 64 + 8, dtype=torch.int32, device="cuda")
    m.dispatch_topk_reduce(act.data_ptr(), res.data_ptr(), n, k, in_off, out_off)
    torch.cuda.synchronize()
    return res.cpu().numpy().view(np.uint32), res


def _cases():
    rng = np.random.default_rng(123)
    yield "vocab_normal", (rng.standard_normal(VOCAB) * 3).astype(np.float16), 32, 0
    yield "vocab_ties", rng.integers(-30, 8, VOCAB).astype(np.float16), 32, 0
    yield "vocab_all_equal", np.full(VOCAB, 1.5, np.float16), 32, 0
    yield "vocab_k1_ties", rng.integers(0, 3, VOCAB).astype(np.float16), 1, 0
    yield "vocab_k8", (rng.standard_normal(VOCAB) * 8).astype(np.float16), 8, 0
    yield "ascending", (np.arange(VOCAB, dtype=np.float32) / 4).astype(np.float16), 32, 0
    yield "descending", (-np.arange(VOCAB, dtype=np.float32) / 64).astype(np.float16), 32, 0
    sp = (rng.standard_normal(4099)).astype(np.float16)
    sp[rng.integers(0, 4099, 40)] = np.nan
    sp[rng.integers(0, 4099, 40)] = -np.inf
    sp[[11, 2000]] = np.inf
    yield "special_odd", sp, 32, 2
    for n in (0, 1, 3, 31, 33, 511, 512, 513, 16385):
        yield f"small_{n}", rng.integers(-4, 4, n + 4).astype(np.float16), 32, 4
    yield "k40_clamped", (rng.standard_normal(VOCAB)).astype(np.float16), 40, 0
    # ties among the top values inside one reference thread (words t, t+256, ..)
    x = (rng.standard_normal(VOCAB) * 2).astype(np.float16)
    a = int(rng.integers(0, VOCAB // 2)) & ~1
    for d in (0, 1, 512, 1024 * 7 + 1):           # same thread: (i >> 1) % 256 equal
        x[a + d] = 12.5
    x[a + 3] = 12.5                                 # another thread, same value
    yield "thread_tie", x, 32, 0
    x = (rng.standard_normal(VOCAB) * 2).astype(np.float16)
    x[rng.choice(VOCAB, 40, replace=False)] = 11.0  # ties spread over threads
    yield "spread_tie", x, 32, 0
    x = (rng.standard_normal(VOCAB)).astype(np.float16)
    x[rng.choice(VOCAB, 1500, replace=False)] = 9.0  # many gathered, under the cap
    yield "near_cap", x, 32, 0
    x = (rng.standard_normal(VOCAB)).astype(np.float16)
    x[rng.choice(VOCAB, 2100, replace=False)] = 9.0  # over the cap: every heap replayed
    yield "over_cap", x, 32, 0
    x = np.full(VOCAB, -np.inf, np.float16)
    x[rng.choice(VOCAB, 20, replace=False)] = rng.standard_normal(20)
    yield "few_finite", x, 32, 0
    x = -np.abs(rng.standard_normal(VOCAB)).astype(np.float16) - np.float16(1)
    z = rng.choice(VOCAB, 60, replace=False)
    x[z[:30]] = 0.0
    x[z[30:]] = -0.0
    yield "signed_zeros", x, 32, 0
    # more than 19 groups of 8 per thread: the groups are loaded in two rounds
    # and the gather re-reads them (group maxima from LDS, then recomputed)
    yield "two_rounds", (rng.standard_normal(200003) * 3).astype(np.float16), 32, 0
    x = rng.integers(-20, 6, 330007).astype(np.float16)
    yield "three_rounds_ties", x, 32, 0


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(range(len(list(_cases())))))
def test_topk_matches_oracle(cuda, case):
    name, x, k, in_off = list(_cases())[case]
    n = x.size - in_off if not name.startswith("small_") else x.size - 4
    out_off = 3
    _say(f"[topk] {name} n={n} k={k} in_off={in_off}")
    x16 = np.ascontiguousarray(x).view(np.uint16)
    _, _, want = _run_oracle(x16, k, in_off=in_off, out_off=out_off, n=n)
    m = _model()
    got, _ = _gpu(m, x16, k, in_off, out_off, n)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{name}: {bad.size} words differ at {bad[:8]}: got {got[bad[:8]]} want {want[bad[:8]]}"
    m.close()


@pytest.mark.gpu
def test_topk_readback_and_repeat(cuda):
    """Two calls in a row on one model (scratch reuse), read back as wait_topk_readback."""
    _say("[topk] readback")
    rng = np.random.default_rng(77)
    m = _model()
    for n, k in ((VOCAB, 32), (1000, 4)):
        x16 = rng.integers(-100, 100, n).astype(np.float16).view(np.uint16)
        wv, wi, _ = _run_oracle(x16, k)
        _, res = _gpu(m, x16, k, 0, 0, n)
        vals, idx = m.wait_topk_readback(res.data_ptr(), 0, k)
        assert np.array_equal(vals.view(np.uint32), wv.view(np.uint32)) and np.array_equal(idx, wi)
    m.close()


@pytest.mark.gpu
def test_topk_rejects_bad_args(cuda):
    import torch
    from bonsai_pot_amd.errors import PotError
    m = _model()
    act = torch.zeros(64, dtype=torch.int16, device="cuda")
    res = torch.zeros(64, dtype=torch.int32, device="cuda")
    with pytest.raises(PotError):
        m.dispatch_topk_reduce(act.data_ptr(), res.data_ptr(), 10, 4, 1, 0)   # odd in_offset
    with pytest.raises(PotError):
        m.dispatch_topk_reduce(0, res.data_ptr(), 10, 4, 0, 0)
    with pytest.raises(PotError):
        m.wait_topk_readback(res.data_ptr(), 0, 33)
    m.close()
