"""Launch-size limits of the prefill path: a call whose grid would exceed
HIP's 65535 limit in y or z fails with BP_ERR_CONFIG (ConfigError) before any
launch, and the call just below the limit still runs."""
import pytest

from bonsai_pot_amd import Model, layout
from bonsai_pot_amd.errors import ConfigError

pytestmark = pytest.mark.gpu


def test_prefill_step_grid_limit_is_a_config_error(cuda, monkeypatch):
    import torch
    # one KV head (kv_dim 128) so that a cache of ~2.1 M rows is small (0.3 GB
    # per buffer, 1.4 GB of image)
    cfg = layout.Config(n_layer=1, n_head=4, n_kv_head=1)
    max_seq = 2_100_100
    pos_bad = 2_097_100    # preparation pass over the image: 2 * 32768 + 4 blocks in y > 65535
    pos_ok = 64 * 32765 - 1   # 2 * ceil((pos + 1) / 64) + 4 = 65534
    print("grid limit: model max_seq", max_seq, flush=True)
    # the image path (the 32x32 kernel; a single token would otherwise take
    # the key-split kernel, which reads the cache directly and builds no image)
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", "2")
    model = Model(cfg, max_seq)
    try:
        model.set_stream(torch.cuda.current_stream().cuda_stream)
        n = cfg.q_dim + 2 * cfg.kv_dim + cfg.q_dim
        act = torch.zeros(n, device="cuda", dtype=torch.float16)
        w = torch.ones(2 * cfg.head_dim, device="cuda", dtype=torch.float16)
        k_off, v_off, out_off = cfg.q_dim, cfg.q_dim + cfg.kv_dim, cfg.q_dim + 2 * cfg.kv_dim

        def step(pos):
            model.dispatch_attention_prefill_step(act.data_ptr(), w.data_ptr(), 0, k_off, v_off, out_off, 0, 128, 0,
                                                  pos, 1)
        with pytest.raises(ConfigError, match="grid limits"):
            step(pos_bad)
        step(pos_ok)
        torch.cuda.synchronize()
        # the plain dispatch (dequantization grid: one per 64-row chunk) fits at pos_bad
        model.dispatch_attention(act.data_ptr(), 0, out_off, 0, pos_bad, 1, 1)
        torch.cuda.synchronize()
        assert torch.isfinite(act[out_off:out_off + cfg.q_dim].float()).all()
    finally:
        model.close()
    # default layout: the key-split kernel, no image, so pos_bad runs
    monkeypatch.delenv("BP_PREFILL_HEADS_PER_WAVE")
    model = Model(cfg, max_seq)
    try:
        model.set_stream(torch.cuda.current_stream().cuda_stream)
        act.zero_()
        model.dispatch_attention_prefill_step(act.data_ptr(), w.data_ptr(), 0, k_off, v_off, out_off, 0, 128, 0,
                                              pos_bad, 1)
        torch.cuda.synchronize()
        assert torch.isfinite(act[out_off:out_off + cfg.q_dim].float()).all()
        print("grid limit: ok", flush=True)
    finally:
        model.close()
