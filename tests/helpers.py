"""Shared scenario builder for oracle-vs-HIP tests.

A Scenario holds, as host numpy arrays, everything one call of the attention
path reads: the f16 activation buffer `act` with regions q / k_cur / v_cur /
attn_out (element offsets like the reference's ActLayout), the f16 norm
weights, the f16 RoPE table and the two KV byte buffers. The same bits are
fed to the CPU oracle and (through torch device memory) to the HIP library.
"""
import ctypes
import math

import numpy as np

import oracle as orc
from bonsai_pot_amd.layout import Config, kv_buffer_bytes, kv_layer_offsets

TOL_MAX_ABS = 2e-3      # attention output vs f32-softmax oracle
TOL_REL_L2 = 1e-3
# (what, max_abs, rel_l2, max_ulp, n_off, n_big) of every attention comparison
# in this process. Over the n_big outputs of magnitude >= ULP_MIN_MAG (where an
# f16 ulp, >= 2^-12, is well above the kernels' error before the f16 store, so
# that the distance isolates that error from the store's own rounding):
# max_ulp is the largest distance, in f16 units in the last place, of an
# output from f16(oracle f32), n_off the number of outputs not equal to it.
# The session summary (tests/conftest.py) prints them with their margin to the
# bar.
MARGINS = []
ULP_MIN_MAG = 0.25


def f16_ulp_distance(got, want) -> np.ndarray:
    """Distance in f16 ulps (steps along the f16 number line, across zero) of
    each f16 value `got` from f16(want) (round to nearest even)."""
    def order(x):
        b = np.asarray(x, np.float32).astype(np.float16).view(np.uint16).astype(np.int64)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(order(got) - order(want))


class Scenario:
    def __init__(self, cfg: Config, max_seq: int, m_tokens: int, seed: int = 0,
                 w_mean: float = 1.0, w_std: float = 0.0, with_q: bool = True):
        self.cfg, self.max_seq, self.m = cfg, max_seq, m_tokens
        rng = np.random.default_rng(seed)
        # act layout: q [m, q_dim] | k_cur [m, kv_dim] | v_cur [m, kv_dim] | out [m, q_dim]
        # (with_q=False: cache-filling scenario, no q / out regions)
        mq = m_tokens if with_q else 0
        self.q_off = 0
        self.k_off = mq * cfg.q_dim
        self.v_off = self.k_off + m_tokens * cfg.kv_dim
        self.out_off = self.v_off + m_tokens * cfg.kv_dim
        n = self.out_off + mq * cfg.q_dim
        vals = rng.standard_normal(n, dtype=np.float32).astype(np.float16)
        vals[self.out_off:] = 0
        self.act = vals.view(np.uint16).copy()
        w = (w_mean + w_std * rng.standard_normal(2 * cfg.head_dim)).astype(np.float16)
        self.w_norms = w.view(np.uint16).copy()       # [w_q_norm (128) | w_k_norm (128)]
        self.w_q_off, self.w_k_off = 0, cfg.head_dim
        _, self.rope = orc.rope_table(cfg.head_dim, cfg.rope_freq_base, max_seq)
        nbytes = kv_buffer_bytes(cfg.n_layer, cfg.kv_dim, max_seq)
        self.kv_k = np.zeros(nbytes, np.uint8)
        self.kv_v = np.zeros(nbytes, np.uint8)

    # -- oracle calls (reference Params) -------------------------------------------
    def layer_offsets(self, il):
        return kv_layer_offsets(self.cfg.n_layer, self.cfg.kv_dim, self.max_seq, il)

    def oracle_writeback(self, il, pos_base, m=None, k_off=None, v_off=None, w_k_off=None):
        m = self.m if m is None else m
        d_word, qs_byte = self.layer_offsets(il)
        p = orc.KvWritebackParams(
            k_cur_off=self.k_off if k_off is None else k_off,
            v_cur_off=self.v_off if v_off is None else v_off,
            w_k_norm_off=self.w_k_off if w_k_off is None else w_k_off, rope_offset=0,
            dst_d_word_offset=d_word, dst_qs_byte_offset=qs_byte, pos_base=pos_base,
            kv_dim=self.cfg.kv_dim, nb_per_row=self.cfg.kv_dim // 32, eps=self.cfg.rms_eps)
        orc.kv_writeback_fused(p, self.act, self.w_norms, self.rope, self.kv_k, self.kv_v,
                               self.cfg.n_kv_head, m)

    def oracle_q_norm_rope(self, pos_base, m=None):
        p = orc.QNormRopeParams(q_off=self.q_off, w_q_norm_off=self.w_q_off, rope_offset=0,
                                pos_base=pos_base, q_dim=self.cfg.q_dim, eps=self.cfg.rms_eps)
        orc.q_norm_rope_fused(p, self.act, self.w_norms, self.rope, self.cfg.n_head,
                              self.m if m is None else m)

    def attn_params(self, il, pos, m, is_prefill):
        d_word, qs_byte = self.layer_offsets(il)
        c = self.cfg
        return orc.AttnParams(head_dim=c.head_dim, n_head=c.n_head, n_kv_head=c.n_kv_head,
                              pos=pos, kv_stride=c.kv_dim, q_offset=self.q_off,
                              k_d_word_offset=d_word, k_qs_byte_offset=qs_byte,
                              v_d_word_offset=d_word, v_qs_byte_offset=qs_byte,
                              out_offset=self.out_off, scale=1.0 / math.sqrt(c.head_dim),
                              m_tokens=m, is_prefill=1 if is_prefill else 0)

    def oracle_attention(self, il, pos, is_prefill=True, tokens=None, m=None):
        p = self.attn_params(il, pos, self.m if m is None else m, is_prefill)
        return orc.attention(p, self.act, self.kv_k, self.kv_v, tokens)

    def oracle_decode(self, il, pos):
        """Reference split/merge decode at step position pos (pos+1 rows)."""
        d_word, qs_byte = self.layer_offsets(il)
        c = self.cfg
        cur = pos + 1
        p = orc.AttnSplitParams(head_dim=c.head_dim, n_head=c.n_head, n_kv_head=c.n_kv_head,
                                pos=cur, kv_stride=c.kv_dim, q_offset=self.q_off,
                                k_d_word_offset=d_word, k_qs_byte_offset=qs_byte,
                                v_d_word_offset=d_word, v_qs_byte_offset=qs_byte,
                                n_chunks_active=(cur + 15) // 16,
                                scale=1.0 / math.sqrt(c.head_dim), out_offset=self.out_off)
        return orc.attention_split_merge(p, self.act, self.kv_k, self.kv_v)


# ---- device side (torch memory as plumbing) -------------------------------------
def hip_runtime():
    """The HIP runtime the library itself is linked against (dlsym through the
    library handle searches its dependencies)."""
    from bonsai_pot_amd import lib
    f = lib.hipMemcpy
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return lib


def d2h(ptr: int, nbytes: int) -> np.ndarray:
    """Synchronous device -> host copy of raw device memory."""
    import torch
    torch.cuda.synchronize()
    out = np.empty(nbytes, np.uint8)
    rc = hip_runtime().hipMemcpy(out.ctypes.data, ptr, nbytes, 2)
    assert rc == 0, f"hipMemcpy D2H failed: {rc}"
    return out


def h2d(ptr: int, host: np.ndarray) -> None:
    import torch
    torch.cuda.synchronize()
    host = np.ascontiguousarray(host)
    rc = hip_runtime().hipMemcpy(ptr, host.ctypes.data, host.nbytes, 1)
    assert rc == 0, f"hipMemcpy H2D failed: {rc}"


class DeviceScenario:
    """Uploads a Scenario's act / w_norms into torch device memory and creates a
    Model whose KV cache starts as the scenario's (usually zero) KV bytes."""

    def __init__(self, sc: Scenario, upload_kv: bool = False):
        import torch
        from bonsai_pot_amd import Model
        self.sc = sc
        self.act = torch.from_numpy(sc.act.view(np.int16).copy()).cuda()
        self.w = torch.from_numpy(sc.w_norms.view(np.int16).copy()).cuda()
        self.model = Model(sc.cfg, sc.max_seq)
        self.model.set_stream(torch.cuda.current_stream().cuda_stream)
        self.kv_k, self.kv_v, self.kv_bytes = self.model.kv_buffers()
        if upload_kv:
            h2d(self.kv_k, sc.kv_k)
            h2d(self.kv_v, sc.kv_v)

    def act_host(self) -> np.ndarray:
        import torch
        torch.cuda.synchronize()
        return self.act.cpu().numpy().view(np.uint16)

    def kv_host(self):
        return d2h(self.kv_k, self.kv_bytes), d2h(self.kv_v, self.kv_bytes)

    def writeback(self, il, pos_base, m=None):
        sc = self.sc
        self.model.dispatch_kv_writeback_fused(self.act.data_ptr(), self.w.data_ptr(), sc.k_off,
                                               sc.v_off, sc.w_k_off, il, pos_base,
                                               sc.m if m is None else m)

    def q_norm_rope(self, pos_base, m=None):
        sc = self.sc
        self.model.dispatch_q_norm_rope_fused(self.act.data_ptr(), self.w.data_ptr(), sc.q_off,
                                              sc.w_q_off, pos_base, sc.m if m is None else m)

    def attention(self, il, pos, is_prefill=True, m=None):
        sc = self.sc
        self.model.dispatch_attention(self.act.data_ptr(), sc.q_off, sc.out_off, il, pos,
                                      sc.m if m is None else m, is_prefill)

    def decode(self, il, pos):
        sc = self.sc
        self.model.dispatch_attention_decode(self.act.data_ptr(), sc.q_off, sc.out_off, il, pos)

    def decode_step(self, il, pos):
        """Fused q_norm_rope + kv_writeback + decode attention for token 0 of the scenario."""
        sc = self.sc
        self.model.dispatch_attention_decode_step(self.act.data_ptr(), self.w.data_ptr(), sc.q_off,
                                                  sc.k_off, sc.v_off, sc.out_off, sc.w_q_off,
                                                  sc.w_k_off, il, pos)

    def out_f32(self, m=None) -> np.ndarray:
        sc = self.sc
        m = sc.m if m is None else m
        a = self.act_host()
        return orc.f16_bits_to_f32(a[sc.out_off:sc.out_off + m * sc.cfg.q_dim]).reshape(m, -1)


def assert_attn_close(got: np.ndarray, want: np.ndarray, what: str = "attention"):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    max_abs = float(err.max())
    rel_l2 = float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))
    big = np.abs(want) >= ULP_MIN_MAG
    ulp = f16_ulp_distance(got[big], want[big])
    MARGINS.append((what, max_abs, rel_l2, int(ulp.max(initial=0)), int(np.count_nonzero(ulp)), int(big.sum())))
    assert max_abs <= TOL_MAX_ABS and rel_l2 <= TOL_REL_L2, (
        f"{what}: max_abs {max_abs:.3e} (<= {TOL_MAX_ABS}), rel_l2 {rel_l2:.3e} (<= {TOL_REL_L2}) "
        f"worst at {np.unravel_index(int(err.argmax()), err.shape)}")
    return max_abs, rel_l2


def write_outlier_rows(sc: Scenario, il: int, n_rows: int, seed: int, frac: float = 0.01):
    """Oracle-written cache rows [0, n_rows) of layer il from an independent
    seeded K/V scenario, with `frac` of the rows' K scaled x8 before
    quantization (a w_k_norm of 8.0 for those rows, exact in f16) — the
    softmax max-tracking stress of BASELINE configs[4]. Returns the rows."""
    cfg = sc.cfg
    pre = Scenario(cfg, sc.max_seq, n_rows, seed=seed, with_q=False)
    pre.kv_k, pre.kv_v = sc.kv_k, sc.kv_v
    pre.oracle_writeback(il, 0)
    rng = np.random.default_rng(seed + 1)
    rows = rng.choice(n_rows, size=max(1, int(n_rows * frac)), replace=False)
    big = Scenario(cfg, sc.max_seq, 1, seed=0, with_q=False)
    big.w_norms = np.concatenate([pre.w_norms, np.full(128, np.float16(8.0)).view(np.uint16)])
    big.kv_k, big.kv_v = sc.kv_k, sc.kv_v
    for r in rows:
        big.act[big.k_off:big.k_off + cfg.kv_dim] = pre.act[pre.k_off + r * cfg.kv_dim:
                                                            pre.k_off + (r + 1) * cfg.kv_dim]
        big.act[big.v_off:big.v_off + cfg.kv_dim] = pre.act[pre.v_off + r * cfg.kv_dim:
                                                            pre.v_off + (r + 1) * cfg.kv_dim]
        big.oracle_writeback(il, int(r), m=1, w_k_off=256)
    return rows
