"""HIP graph replays of the library's entry points, the way bench.py times
every figure: each case runs its calls once eagerly, then captures the same
calls into a graph on a side stream and replays it several times. Before every
replay the act buffer is restored by an eager copy (the fused steps normalize q
in place) and the caches are left as the eager run wrote them (every call
rewrites the same rows with the same bytes); after it, the whole act buffer and
the K/V cache bytes must equal the eager run's bit for bit. The library records
no memset nodes (its scratch, the split-K partials, is written before it is
read), so every replay must reproduce the first one.
"""
import sys

import numpy as np
import pytest

from bonsai_pot_amd import layout
from helpers import DeviceScenario, Scenario

pytestmark = pytest.mark.gpu

N_REPLAYS = 4


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _scenario(m, pos, seed, n_layer=2, rows=None):
    """Scenario of m tokens at pos, cache rows [0, rows) (default pos) of every
    layer oracle-written from independent seeded K/V."""
    cfg = layout.Config(n_layer=n_layer)
    sc = Scenario(cfg, max_seq=pos + m + 5, m_tokens=m, seed=seed, w_std=0.1)
    rows = pos if rows is None else rows
    for il in range(n_layer):
        if rows:
            pre = Scenario(cfg, sc.max_seq, rows, seed=seed + 1 + il, with_q=False)
            pre.kv_k, pre.kv_v = sc.kv_k, sc.kv_v
            pre.oracle_writeback(il, 0)
    return sc


def _check_replays(dev, body, what):
    import torch
    act0 = dev.act.clone()
    body()
    torch.cuda.synchronize()
    act_ref = dev.act_host().copy()
    k_ref, v_ref = dev.kv_host()

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        dev.model.set_stream(side.cuda_stream)
        with torch.cuda.graph(graph, stream=side):
            body()
    dev.model.set_stream(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()

    for r in range(N_REPLAYS):
        dev.act.copy_(act0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        act = dev.act_host()
        k, v = dev.kv_host()
        assert np.array_equal(act, act_ref), f"{what}: replay {r}: act differs at {np.flatnonzero(act != act_ref)[:8]}"
        assert np.array_equal(k, k_ref), f"{what}: replay {r}: K cache bytes differ"
        assert np.array_equal(v, v_ref), f"{what}: replay {r}: V cache bytes differ"
    # the model still runs eagerly on its own stream afterwards
    dev.act.copy_(act0)
    body()
    assert np.array_equal(dev.act_host(), act_ref), f"{what}: eager call after the replays differs"


@pytest.mark.parametrize("wide_min", ["2147483648", "0"])
def test_graph_decode_steps(cuda, monkeypatch, wide_min):
    """Two layers of the fused decode step at pos 4096 (both split layouts), and
    the plain decode entry point, in one graph."""
    monkeypatch.setenv("BP_DECODE_WIDE_MIN_ROWS", wide_min)
    _say(f"[graph] decode steps wide_min={wide_min}")
    pos = 4096
    sc = _scenario(1, pos, seed=5100)
    dev = DeviceScenario(sc, upload_kv=True)

    def body():
        dev.decode_step(0, pos)
        dev.decode_step(1, pos)
        dev.decode(1, pos)
    _check_replays(dev, body, f"decode wide_min={wide_min}")


@pytest.mark.parametrize("entry", ["step", "dispatch"])
@pytest.mark.parametrize("m,pos", [(512, 0), (2048, 0), (64, 4096), (300, 64)])
def test_graph_prefill(cuda, m, pos, entry):
    """The fused prefill step (preparation pass + attention kernel) and the
    plain attention dispatch (image pass + attention kernel): the 16x16
    kernels (512 tokens), prefill32_kernel (2048), the key-split kernel and
    its merge pass (64 tokens on 4096 rows), and a chunk that mixes cache rows
    and new rows (300 on 64)."""
    _say(f"[graph] prefill {entry} m={m} pos={pos}")
    # the dispatch attends rows [0, pos + m): all of them written beforehand
    sc = _scenario(m, pos, seed=5200 + m + pos, rows=pos if entry == "step" else pos + m)
    dev = DeviceScenario(sc, upload_kv=True)

    def step():
        dev.model.dispatch_attention_prefill_step(dev.act.data_ptr(), dev.w.data_ptr(), sc.q_off, sc.k_off,
                                                  sc.v_off, sc.out_off, sc.w_q_off, sc.w_k_off, 1, pos, m)

    def dispatch():
        dev.attention(1, pos, is_prefill=True)
    _check_replays(dev, step if entry == "step" else dispatch, f"prefill {entry} m={m} pos={pos}")
