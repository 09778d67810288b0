"""KvSnapshot capture / apply through the device (src/kv_snapshot.rs:203-372):
the payload read back from the HIP KV cache equals the oracle's payload of the
same cache bytes, a BONSAIKV v1 round trip restores exactly rows < pos of
every layer into a fresh model, and rows >= pos stay untouched."""
import sys

import numpy as np
import pytest

import oracle as orc
from helpers import DeviceScenario, Scenario


@pytest.mark.gpu
@pytest.mark.parametrize("pos", [1, 37, 64])
def test_snapshot_capture_apply_roundtrip(cuda, pos):
    print(f"[snapshot] pos={pos}", flush=True)
    sys.stdout.flush()
    from bonsai_pot_amd import layout
    from bonsai_pot_amd.snapshot import KvSnapshot
    cfg = layout.Config(n_layer=3)
    max_seq = 80
    sc = Scenario(cfg, max_seq=max_seq, m_tokens=64, seed=31, with_q=False)
    dev = DeviceScenario(sc)
    for il in range(cfg.n_layer):
        dev.writeback(il, 0)
    k, v = dev.kv_host()
    snap = KvSnapshot.capture(dev.model, pos)
    want = orc.snapshot_capture(cfg.n_layer, cfg.kv_dim, max_seq, pos, k, v)
    assert np.array_equal(np.frombuffer(snap.payload, np.uint8), want)

    blob = snap.to_bytes()
    sc2 = Scenario(cfg, max_seq=max_seq, m_tokens=1, seed=32, with_q=False)
    rng = np.random.default_rng(pos)
    sc2.kv_k[:] = rng.integers(0, 256, sc2.kv_k.size, dtype=np.uint8)
    sc2.kv_v[:] = rng.integers(0, 256, sc2.kv_v.size, dtype=np.uint8)
    dev2 = DeviceScenario(sc2, upload_kv=True)
    KvSnapshot.from_bytes(blob).apply(dev2.model)
    k2, v2 = dev2.kv_host()
    wk, wv = sc2.kv_k.copy(), sc2.kv_v.copy()
    orc.snapshot_apply(cfg.n_layer, cfg.kv_dim, max_seq, pos, want, wk, wv)
    assert np.array_equal(k2, wk) and np.array_equal(v2, wv)
    dev.model.close()
    dev2.model.close()
