"""ctypes binding of ``libbonsai_pot_hip.so`` and the :class:`Model` wrapper.

:class:`Model` mirrors the attention part of the reference's ``Model``
(src/model.rs) and the dispatch helpers of src/forward.rs, one method per
C entry point; every failing status raises the matching :class:`PotError`.
"""
import ctypes
import os

from .errors import BP_OK, error_for
from .layout import Config

_HERE = os.path.dirname(os.path.abspath(__file__))
library_path = os.environ.get("BONSAI_POT_HIP_LIB") or os.path.join(os.path.dirname(_HERE), "lib",
                                                                   "libbonsai_pot_hip.so")

if not os.path.exists(library_path):
    raise ImportError(
        f"{library_path} is missing: build the HIP library first "
        "(python bonsai-pot_amd/build.py or __graft_entry__.build()); there is no CPU fallback")



def _preload_torch_hip_runtime() -> None:
    """One HIP runtime per process. PyTorch-ROCm wheels bundle their own
    libamdhip64 (soname libamdhip64.so.7) and load it by file name; if this
    library were loaded first it would bring in /opt/rocm's copy and the process
    would hold two runtimes (separate device/stream state). Loading torch's copy
    first, RTLD_GLOBAL, makes both resolve to the same runtime. Nothing is
    imported from torch."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    for loc in spec.submodule_search_locations:
        cand = os.path.join(loc, "lib", "libamdhip64.so")
        if os.path.exists(cand):
            ctypes.CDLL(cand, mode=ctypes.RTLD_GLOBAL)
            return


_preload_torch_hip_runtime()
lib = ctypes.CDLL(library_path)


class MatvecRange(ctypes.Structure):
    """bp_matvec_range: one Q1_0 tensor of a fused normed matvec."""
    _fields_ = [("d_offset", ctypes.c_uint32), ("qs_offset", ctypes.c_uint32), ("n", ctypes.c_uint32),
                ("output_offset", ctypes.c_uint32)]


class _Config(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_uint32), ("n_head", ctypes.c_uint32),
                ("n_kv_head", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("rms_eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float)]


_u32, _u64, _vp, _i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int32
_SIGS = {
    "bp_model_create": (_i32, [ctypes.POINTER(_Config), _u32, ctypes.c_int, ctypes.POINTER(_vp)]),
    "bp_model_destroy": (None, [_vp]),
    "bp_model_set_stream": (_i32, [_vp, _vp]),
    "bp_model_synchronize": (_i32, [_vp]),
    "bp_model_kv_buffers": (_i32, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_u64)]),
    "bp_model_rope_table": (_i32, [_vp, ctypes.POINTER(_vp)]),
    "bp_model_max_seq": (_u32, [_vp]),
    "bp_kv_layer_offsets": (_i32, [_u32, _u32, _u32, _u32, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "bp_kv_buffer_bytes": (_u64, [_u32, _u32, _u32]),
    "bp_dispatch_q_norm_rope_fused": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "bp_dispatch_kv_writeback_fused": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32]),
    "bp_dispatch_attention_decode": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32]),
    "bp_dispatch_attention_decode_step": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                                  _u32]),
    "bp_dispatch_attention": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32]),
    "bp_dispatch_attention_prefill_step": (_i32, [_vp, _vp, _vp] + [_u32] * 9),
    "bp_dispatch_matvec_q1_0": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32]),
    "bp_dispatch_matvec_q1_0_silu": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32]),
    "bp_dispatch_matvec_q1_0_fused_normed": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                                     ctypes.POINTER(MatvecRange)]),
    "bp_dispatch_quantize_act": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32]),
    "bp_dispatch_matmul_q1_0": (_i32, [_vp, _vp, _vp, _vp] + [_u32] * 9),
    "bp_dispatch_topk_reduce": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "bp_topk_readback": (_i32, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "bp_kv_snapshot_payload_bytes": (_u64, [_u32, _u32, _u32]),
    "bp_kv_snapshot_capture": (_i32, [_vp, _u32, _vp, _u64]),
    "bp_kv_snapshot_apply": (_i32, [_vp, _u32, _vp, _u64]),
    "bp_attention_decode_noalloc": (_i32, [ctypes.POINTER(_Config), _vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32,
                                            _vp]),
    "bp_check_device": (_i32, [_vp]),
    "bp_debug_lose_device": (_i32, [_vp]),
    "bp_last_error": (ctypes.c_char_p, []),
    "bp_status_name": (ctypes.c_char_p, [_i32]),
}
# Measurement hooks of include/bonsai_pot_hip_bench.h, exported only by the
# bench build (lib/libbonsai_pot_hip_bench.so, which bench.py loads).
_BENCH_SIGS = {
    "bp_debug_prefill_prep": (_i32, [_vp, _vp, _vp] + [_u32] * 9),
    "bp_debug_read_floor": (_i32, [_vp, _u64, _vp, _u32, _vp]),
    "bp_debug_mfma_rate": (_i32, [_vp, _u32, _u32, _u32, _vp]),
}
EXPORTED_SYMBOLS = tuple(_SIGS)
BENCH_SYMBOLS = tuple(_BENCH_SIGS)
for _name, (_res, _args) in list(_SIGS.items()) + [kv for kv in _BENCH_SIGS.items() if hasattr(lib, kv[0])]:
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def _check(status: int) -> None:
    if status != BP_OK:
        msg = lib.bp_last_error().decode(errors="replace")
        name = lib.bp_status_name(status).decode()
        raise error_for(status, f"{name}: {msg}")


class Model:
    """Device-side state of the attention path for one model on one GPU."""

    def __init__(self, cfg: Config, max_seq: int, device: int = 0):
        self.cfg = cfg
        self.max_seq = max_seq
        c = _Config(cfg.n_layer, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.rms_eps,
                    cfg.rope_freq_base)
        h = _vp()
        _check(lib.bp_model_create(ctypes.byref(c), max_seq, device, ctypes.byref(h)))
        self._h = h

    # -- lifetime ------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            lib.bp_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    # -- buffers ---------------------------------------------------------------
    def set_stream(self, stream_ptr: int) -> None:
        _check(lib.bp_model_set_stream(self._h, stream_ptr))

    def synchronize(self) -> None:
        _check(lib.bp_model_synchronize(self._h))

    def kv_buffers(self):
        """(kv_k device address, kv_v device address, bytes of each)."""
        k, v, n = _vp(), _vp(), _u64()
        _check(lib.bp_model_kv_buffers(self._h, ctypes.byref(k), ctypes.byref(v), ctypes.byref(n)))
        return k.value, v.value, n.value

    def rope_table(self) -> int:
        p = _vp()
        _check(lib.bp_model_rope_table(self._h, ctypes.byref(p)))
        return p.value

    def layer_offsets(self, il: int):
        d, q = _u64(), _u64()
        _check(lib.bp_kv_layer_offsets(self.cfg.n_layer, self.cfg.kv_dim, self.max_seq, il,
                                       ctypes.byref(d), ctypes.byref(q)))
        return d.value, q.value

    # -- dispatch helpers (src/forward.rs) -------------------------------------
    def dispatch_q_norm_rope_fused(self, act: int, w_norms: int, q_off: int, w_q_norm_off: int,
                                   pos_base: int, m_tokens: int) -> None:
        _check(lib.bp_dispatch_q_norm_rope_fused(self._h, act, w_norms, q_off, w_q_norm_off,
                                                 pos_base, m_tokens))

    def dispatch_kv_writeback_fused(self, act: int, w_norms: int, k_cur_off: int, v_cur_off: int,
                                    w_k_norm_off: int, layer_il: int, pos_base: int,
                                    m_tokens: int) -> None:
        _check(lib.bp_dispatch_kv_writeback_fused(self._h, act, w_norms, k_cur_off, v_cur_off,
                                                  w_k_norm_off, layer_il, pos_base, m_tokens))

    def dispatch_attention_decode(self, act: int, q_off: int, out_off: int, layer_il: int,
                                  pos: int) -> None:
        _check(lib.bp_dispatch_attention_decode(self._h, act, q_off, out_off, layer_il, pos))

    def dispatch_attention_decode_step(self, act: int, w_norms: int, q_off: int, k_cur_off: int,
                                       v_cur_off: int, out_off: int, w_q_norm_off: int,
                                       w_k_norm_off: int, layer_il: int, pos: int) -> None:
        """q_norm_rope + kv_writeback + decode attention for one token, fused."""
        _check(lib.bp_dispatch_attention_decode_step(self._h, act, w_norms, q_off, k_cur_off,
                                                     v_cur_off, out_off, w_q_norm_off,
                                                     w_k_norm_off, layer_il, pos))

    def dispatch_attention(self, act: int, q_off: int, out_off: int, layer_il: int, pos: int,
                           m_tokens: int, is_prefill: bool) -> None:
        _check(lib.bp_dispatch_attention(self._h, act, q_off, out_off, layer_il, pos, m_tokens,
                                         1 if is_prefill else 0))

    def dispatch_attention_prefill_step(self, act: int, w_norms: int, q_off: int, k_cur_off: int,
                                        v_cur_off: int, out_off: int, w_q_norm_off: int,
                                        w_k_norm_off: int, layer_il: int, pos: int,
                                        m_tokens: int) -> None:
        """q_norm_rope + kv_writeback + causal attention for m_tokens tokens, fused."""
        _check(lib.bp_dispatch_attention_prefill_step(self._h, act, w_norms, q_off, k_cur_off,
                                                      v_cur_off, out_off, w_q_norm_off,
                                                      w_k_norm_off, layer_il, pos, m_tokens))

    def debug_prefill_prep(self, act: int, w_norms: int, q_off: int, k_cur_off: int, v_cur_off: int,
                           out_off: int, w_q_norm_off: int, w_k_norm_off: int, layer_il: int, pos: int,
                           m_tokens: int) -> None:
        """Measurement aid (bench build of the library only): the first launch of
        dispatch_attention_prefill_step alone."""
        _check(lib.bp_debug_prefill_prep(self._h, act, w_norms, q_off, k_cur_off, v_cur_off, out_off,
                                         w_q_norm_off, w_k_norm_off, layer_il, pos, m_tokens))

    # -- Q1_0 decode matvecs (src/forward.rs:212-334) -----------------------------
    # `weights` and `act` are device pointers (ints); w_d / w_qs byte offsets.
    def dispatch_matvec_q1_0(self, weights: int, act: int, k: int, n: int, w_d: int, w_qs: int,
                             in_off: int, out_off: int, accumulate: bool) -> None:
        _check(lib.bp_dispatch_matvec_q1_0(self._h, weights, act, k, n, w_d, w_qs, in_off, out_off,
                                           1 if accumulate else 0))

    def dispatch_matvec_q1_0_silu(self, weights: int, act: int, k: int, n: int, w_d: int, w_qs: int,
                                  gate_off: int, up_off: int, out_off: int, accumulate: bool) -> None:
        _check(lib.bp_dispatch_matvec_q1_0_silu(self._h, weights, act, k, n, w_d, w_qs, gate_off, up_off,
                                                out_off, 1 if accumulate else 0))

    def dispatch_matvec_q1_0_fused_normed(self, weights: int, act: int, w_norms: int, k: int,
                                          input_offset: int, w_norm_off: int, ranges) -> None:
        """ranges: sequence of (d_offset, qs_offset, n, output_offset), 2 or 3 of them."""
        arr = (MatvecRange * max(1, len(ranges)))(*[MatvecRange(*r) for r in ranges])
        _check(lib.bp_dispatch_matvec_q1_0_fused_normed(self._h, weights, act, w_norms, k, input_offset,
                                                        w_norm_off, len(ranges), arr))

    # -- prefill projections (src/forward.rs:415-472) -----------------------------
    def dispatch_quantize_act(self, act: int, acts_q8: int, k: int, m_tokens: int, in_off: int, d_off: int,
                              qs_off: int) -> None:
        _check(lib.bp_dispatch_quantize_act(self._h, act, acts_q8, k, m_tokens, in_off, d_off, qs_off))

    def dispatch_matmul_q1_0(self, weights: int, acts_q8: int, act: int, k: int, n: int, m_tokens: int,
                             w_d: int, w_qs: int, a_d: int, a_qs: int, out_off: int, accumulate: bool) -> None:
        _check(lib.bp_dispatch_matmul_q1_0(self._h, weights, acts_q8, act, k, n, m_tokens, w_d, w_qs, a_d, a_qs,
                                           out_off, 1 if accumulate else 0))

    # -- top-k (src/forward.rs:336-354, :542-568) ---------------------------------
    def dispatch_topk_reduce(self, act: int, result: int, n: int, k: int, in_off: int, out_off: int) -> None:
        _check(lib.bp_dispatch_topk_reduce(self._h, act, result, n, k, in_off, out_off))

    def wait_topk_readback(self, result: int, out_off: int, k: int):
        """(values f32[k], indices u32[k]) after the stream drains, as wait_topk_readback."""
        import numpy as np
        vals = np.zeros(k, np.float32)
        idx = np.zeros(k, np.uint32)
        _check(lib.bp_topk_readback(self._h, result, out_off, k, vals.ctypes.data_as(_vp),
                                    idx.ctypes.data_as(_vp)))
        return vals, idx

    # -- snapshot payload (src/kv_snapshot.rs:203-372) ----------------------------
    def snapshot_payload(self, pos: int) -> bytes:
        n = lib.bp_kv_snapshot_payload_bytes(self.cfg.n_layer, self.cfg.kv_dim, pos)
        buf = ctypes.create_string_buffer(max(n, 1))
        _check(lib.bp_kv_snapshot_capture(self._h, pos, buf, n))
        return buf.raw[:n]

    def apply_payload(self, pos: int, payload: bytes) -> None:
        buf = ctypes.create_string_buffer(bytes(payload), max(len(payload), 1))
        _check(lib.bp_kv_snapshot_apply(self._h, pos, buf, len(payload)))

    # -- device loss (src/model.rs:1733-1751) -----------------------------------
    def check_device(self) -> None:
        _check(lib.bp_check_device(self._h))

    def is_device_lost(self) -> bool:
        return lib.bp_check_device(self._h) != BP_OK

    def _destroy_device_for_test(self) -> None:
        _check(lib.bp_debug_lose_device(self._h))
