"""A second, independent restatement of src/shaders/topk_reduce.wgsl (reference
repository) as a workgroup simulator, to pin the C oracle's tie order.

The oracle (oracle/bp_oracle.c, bpo_topk_reduce) restates the shader in C.
This file restates it again, separately, in the shader's own terms: 256
invocations, one shared `sh_val` / `sh_idx` array pair of 256 x 32 entries,
and the phases between workgroupBarrier() calls. Within one such phase every
invocation of this shader reads and writes only entries no other invocation
touches in that phase (its own 32-entry heap in phases 1 and 2a, the disjoint
compare-swap pairs of one merge stage in phase 2b), so running the
invocations one after another gives the result of any parallel schedule.

Line references are to topk_reduce.wgsl. Which of several equal logits the
reference returns, and in which order, is decided only by these steps (the
strict `>` / `<` comparisons, the heap's sift order and the merge network), so
agreement of two separate restatements on tie-heavy inputs is the check
available for it; nothing executable of the reference runs here.
"""
import zlib

import numpy as np
import pytest

import oracle as orc

WG = 256          # :41
K_MAX = 32        # :42
NEG_INIT = float(np.float32(-1e30))   # :68, an f32 constant


def _sift_down(val, idx, base, size):
    """:47-60 (size K_MAX) and the phase-2a re-sift :107-118 (size active)."""
    i = 0
    while True:
        l = 2 * i + 1
        r = l + 1
        smallest = i
        if l < size and val[base + l] < val[base + smallest]:
            smallest = l
        if r < size and val[base + r] < val[base + smallest]:
            smallest = r
        if smallest == i:
            return
        val[base + i], val[base + smallest] = val[base + smallest], val[base + i]
        idx[base + i], idx[base + smallest] = idx[base + smallest], idx[base + i]
        i = smallest


def _merge_lists(val, idx, a_base, b_base):
    """List a absorbs list b: stage 0 (:141-153), then the strict compare-swap
    stages of stride 16 .. 1 (:156-181)."""
    for i in range(K_MAX):
        bi = K_MAX - 1 - i
        if val[b_base + bi] > val[a_base + i]:
            val[a_base + i] = val[b_base + bi]
            idx[a_base + i] = idx[b_base + bi]
    stride = K_MAX // 2
    while stride > 0:
        for local in range(K_MAX // 2):
            lo = ((local & ~(stride - 1)) << 1) | (local & (stride - 1))
            hi = lo | stride
            vlo, vhi = val[a_base + lo], val[a_base + hi]
            if vhi > vlo:
                ilo = idx[a_base + lo]
                val[a_base + lo], val[a_base + hi] = vhi, vlo
                idx[a_base + lo] = idx[a_base + hi]
                idx[a_base + hi] = ilo
        stride //= 2


def simulate(words_f16: np.ndarray, n: int, in_offset: int, k: int):
    """Returns (values as f32 bit patterns, indices) of the top-min(k, 32)."""
    halves = words_f16.view(np.float16)
    val = [0.0] * (WG * K_MAX)
    idx = [0] * (WG * K_MAX)
    in_word_off = in_offset >> 1
    n_words = (n + 1) >> 1
    # ---- phase 1 (:63-94) and phase 2a (:96-119), per invocation ----
    for tid in range(WG):
        base = tid * K_MAX
        for i in range(K_MAX):
            val[base + i] = NEG_INIT
            idx[base + i] = 0
        w = tid
        while w < n_words:
            word = in_word_off + w
            v0 = float(halves[2 * word])
            v1 = float(halves[2 * word + 1]) if 2 * word + 1 < halves.size else 0.0
            i0 = w << 1
            i1 = i0 + 1
            if v0 > val[base]:
                val[base] = v0
                idx[base] = i0
                _sift_down(val, idx, base, K_MAX)
            if i1 < n:
                if v1 > val[base]:
                    val[base] = v1
                    idx[base] = i1
                    _sift_down(val, idx, base, K_MAX)
            w += WG
        for active_minus1 in range(K_MAX - 1, 0, -1):
            last = base + active_minus1
            val[base], val[last] = val[last], val[base]
            idx[base], idx[last] = idx[last], idx[base]
            _sift_down(val, idx, base, active_minus1)
    # ---- phase 2b (:121-184): pairwise merges, s = 128 .. 1 ----
    # (each stage's invocations touch disjoint pairs of lists, so running the
    # merges pair by pair gives the same entries)
    s = WG // 2
    while s > 0:
        for pair_id in range(s):
            _merge_lists(val, idx, pair_id * K_MAX, (pair_id + s) * K_MAX)
        s //= 2
    kk = min(k, K_MAX)                          # :186-194
    vals = np.array(val[:kk], np.float32).view(np.uint32)
    return vals, np.array(idx[:kk], np.uint32)


def _oracle(x16, k, in_off, n):
    res = np.zeros(64 + 8, np.uint32)
    out = orc.topk_reduce(orc.TopKParams(n=n, in_offset=in_off, out_offset=0, k=k), x16, res)
    kk = min(k, 32)
    return out[:kk], out[kk:2 * kk]


def _case(name, rng, n):
    if name == "few_values":      # heavy ties: 5 distinct values
        return rng.choice(np.array([-1.0, 0.5, 2.0, 3.0, 3.0], np.float16), n)
    if name == "all_equal":
        return np.full(n, np.float16(1.25))
    if name == "ties_at_top":     # distinct background, 100 copies of the maximum
        x = rng.standard_normal(n).astype(np.float16)
        x[rng.choice(n, min(100, n // 2), replace=False)] = np.float16(9.0)
        return x
    if name == "quantized":       # values on a coarse grid: many ties everywhere
        return (np.round(rng.standard_normal(n) * 4) / 4).astype(np.float16)
    if name == "specials":        # NaN, +-inf among ties
        x = rng.choice(np.array([0.0, 1.0, 1.0, 2.0], np.float16), n)
        x[rng.choice(n, 9, replace=False)] = np.float16(np.nan)
        x[rng.choice(n, 5, replace=False)] = np.float16(-np.inf)
        x[rng.choice(n, 3, replace=False)] = np.float16(np.inf)
        return x
    raise ValueError(name)


@pytest.mark.parametrize("name", ["few_values", "all_equal", "ties_at_top", "quantized", "specials"])
@pytest.mark.parametrize("n,k,in_off", [(4099, 32, 0), (1537, 8, 6), (600, 40, 2), (9000, 32, 0), (31, 32, 0)])
def test_oracle_tie_order_matches_independent_simulation(name, n, k, in_off):
    rng = np.random.default_rng(zlib.crc32(f"{name}/{n}".encode()))
    x = np.zeros(in_off + n + 1, np.float16)
    x[in_off:in_off + n] = _case(name, rng, n)
    words = x.view(np.uint16)
    want_v, want_i = simulate(words, n, in_off, k)
    got_v, got_i = _oracle(words, k, in_off, n)
    assert np.array_equal(got_i, want_i), (name, n, k, got_i[:8], want_i[:8])
    assert np.array_equal(got_v, want_v), (name, n, k)


def test_simulation_distinct_is_sorted_topk():
    """The simulator itself against what the mathematics fixes: distinct
    logits give the descending top-k by np.argsort."""
    rng = np.random.default_rng(3)
    pool = np.arange(0x0000, 0x7BFF, dtype=np.uint16)
    x = rng.permutation(np.concatenate([pool, pool[1:] | np.uint16(0x8000)]))[:3001].view(np.float16)
    v, i = simulate(x.view(np.uint16), 3001, 0, 32)
    order = np.argsort(-x.astype(np.float64), kind="stable")[:32]
    assert np.array_equal(i, order)
    assert np.array_equal(v.view(np.float32), x[order].astype(np.float32))


def test_one_entry_merge_closed_form():
    """The kernel merges two lists of one entry each (or an empty first list
    and a one-entry second list) without the network: [x, y] if y <= x and
    [y, x] if y > x, fill after. Checked against the simulator's network for
    equal values, signed zeros, infinities and the -1e30 fill as x."""
    fill = np.float32(-1e30)
    vals = [np.float32(v) for v in (0.0, -0.0, 1.5, -1.5, 65504.0, -65504.0, np.inf, 3.0, 3.0)]
    for x in vals + [fill]:
        for y in vals:
            xi = 0 if x == fill else 1
            val = [x] + [fill] * (K_MAX - 1) + [y] + [fill] * (K_MAX - 1)
            ix = [xi] + [0] * (K_MAX - 1) + [2] + [0] * (K_MAX - 1)
            _merge_lists(val, ix, 0, K_MAX)
            want = [(y, 2), (x, xi)] if y > x else [(x, xi), (y, 2)]
            got = [(val[0], ix[0]), (val[1], ix[1])]
            assert [(np.float32(a).tobytes(), b) for a, b in got] == \
                [(np.float32(a).tobytes(), b) for a, b in want], (x, y, got)
            assert all(v == fill for v in val[2:K_MAX]) and all(i == 0 for i in ix[2:K_MAX])
