"""numpy-facing ctypes wrapper of the CPU oracle (oracle/bp_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker — never by the product path.

Arrays: f16 data is passed as numpy uint16 bit patterns (or float16 arrays,
viewed as uint16); KV buffers are uint8 arrays of the reference byte layout.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# BP_ORACLE_LIB selects another build of the same source (the sanitizer build
# of tests/test_sanitizers.py).
LIB_PATH = os.environ.get("BP_ORACLE_LIB") or os.path.join(HERE, "libbp_oracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


if not os.path.exists(LIB_PATH):
    build()
_lib = ctypes.CDLL(LIB_PATH)

_u32, _u64, _f32, _vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p


class KvWritebackParams(ctypes.Structure):
    """KvWritebackFusedParams, src/model.rs:265-276."""
    _fields_ = [(n, _u32) for n in ("k_cur_off", "v_cur_off", "w_k_norm_off", "rope_offset",
                                     "dst_d_word_offset", "dst_qs_byte_offset", "pos_base",
                                     "kv_dim", "nb_per_row")] + [("eps", _f32)]


class QNormRopeParams(ctypes.Structure):
    """QNormRopeFusedParams, src/model.rs:255-262."""
    _fields_ = [(n, _u32) for n in ("q_off", "w_q_norm_off", "rope_offset", "pos_base",
                                     "q_dim")] + [("eps", _f32)]


class AttnSplitParams(ctypes.Structure):
    """AttnSplitParams (src/model.rs:213-226) + AttnMergeParams.out_offset."""
    _fields_ = [(n, _u32) for n in ("head_dim", "n_head", "n_kv_head", "pos", "kv_stride",
                                     "q_offset", "k_d_word_offset", "k_qs_byte_offset",
                                     "v_d_word_offset", "v_qs_byte_offset", "n_chunks_active")] + \
               [("scale", _f32), ("out_offset", _u32)]


class AttnParams(ctypes.Structure):
    """AttnParams, src/model.rs:195-210."""
    _fields_ = [(n, _u32) for n in ("head_dim", "n_head", "n_kv_head", "pos", "kv_stride",
                                     "q_offset", "k_d_word_offset", "k_qs_byte_offset",
                                     "v_d_word_offset", "v_qs_byte_offset", "out_offset")] + \
               [("scale", _f32), ("m_tokens", _u32), ("is_prefill", _u32)]


class MatvecParams(ctypes.Structure):
    """MatvecParams, src/model.rs:105-114 (without dispatch_x_dim)."""
    _fields_ = [(n, _u32) for n in ("k", "n", "d_offset", "qs_offset", "input_offset",
                                     "output_offset", "accumulate")]


class MatvecSiluParams(ctypes.Structure):
    """MatvecSiluParams, src/model.rs:117-127 (without dispatch_x_dim)."""
    _fields_ = [(n, _u32) for n in ("k", "n", "d_offset", "qs_offset", "gate_offset", "up_offset",
                                     "output_offset", "accumulate")]


class MatvecFusedNormedParams(ctypes.Structure):
    """MatvecFusedNormedParams, src/model.rs:150-169, ranges as arrays."""
    _fields_ = [("k", _u32), ("input_offset", _u32), ("w_norm_off", _u32), ("eps", _f32),
                ("n_ranges", _u32), ("d_offset", _u32 * 3), ("qs_offset", _u32 * 3), ("n", _u32 * 3),
                ("output_offset", _u32 * 3)]


class QuantParams(ctypes.Structure):
    """QuantParams, src/model.rs:172-179 (without dispatch_x_dim)."""
    _fields_ = [(n, _u32) for n in ("k", "m", "input_offset", "d_offset", "qs_offset")]


class MatmulParams(ctypes.Structure):
    """MatmulParams, src/model.rs:182-192."""
    _fields_ = [(n, _u32) for n in ("k", "n", "m", "w_d_offset", "w_qs_offset", "a_d_offset", "a_qs_offset",
                                     "out_offset", "accumulate")]


class TopKParams(ctypes.Structure):
    """TopKParams, src/forward.rs:343-348 (n, in_offset, out_offset, k)."""
    _fields_ = [(n, _u32) for n in ("n", "in_offset", "out_offset", "k")]


def _sig(name, res, args):
    f = getattr(_lib, name)
    f.restype, f.argtypes = res, args
    return f


_f32_to_f16 = _sig("bpo_f32_to_f16", ctypes.c_uint16, [_f32])
_f16_to_f32 = _sig("bpo_f16_to_f32", _f32, [ctypes.c_uint16])
_f32_to_f16_arr = _sig("bpo_f32_to_f16_array", None, [_vp, _vp, ctypes.c_size_t])
_f16_to_f32_arr = _sig("bpo_f16_to_f32_array", None, [_vp, _vp, ctypes.c_size_t])
_rope = _sig("bpo_build_rope_table", None, [_u32, _f32, _u32, _vp, _vp])
_layer_off = _sig("bpo_kv_layer_offsets", None, [_u32, _u32, _u32, _u32, ctypes.POINTER(_u64),
                                                 ctypes.POINTER(_u64)])
_buf_bytes = _sig("bpo_kv_buffer_bytes", _u64, [_u32, _u32, _u32])
_snap_bytes = _sig("bpo_snapshot_payload_bytes", _u64, [_u32, _u32, _u32])
_snap_off = _sig("bpo_snapshot_payload_offset", _u64, [_u32, _u32, _u32, _u32, _u32, _u32])
_snap_cap = _sig("bpo_snapshot_capture", None, [_u32, _u32, _u32, _u32, _vp, _vp, _vp])
_snap_apply = _sig("bpo_snapshot_apply", None, [_u32, _u32, _u32, _u32, _vp, _vp, _vp])
_quant = _sig("bpo_quantize_q8_0_block", None, [_vp, _vp, _vp])
_kvwb = _sig("bpo_kv_writeback_fused", None, [ctypes.POINTER(KvWritebackParams), _vp, _vp, _vp,
                                             _vp, _vp, _u32, _u32])
_qnr = _sig("bpo_q_norm_rope_fused", None, [ctypes.POINTER(QNormRopeParams), _vp, _vp, _vp, _u32,
                                           _u32])
_split = _sig("bpo_attention_split_merge", None, [ctypes.POINTER(AttnSplitParams), _vp, _vp, _vp,
                                                  _vp, _vp])
_attn = _sig("bpo_attention", None, [ctypes.POINTER(AttnParams), _vp, _vp, _vp, _vp, _u32, _vp,
                                    _vp])
_fill = _sig("bpo_fill_normal_f16", None, [_u64, _f32, _f32, _vp, ctypes.c_size_t])
_quant_act = _sig("bpo_quantize_act_q8_0", None, [ctypes.POINTER(QuantParams), _vp, _vp])
_matmul = _sig("bpo_matmul_q1_0_q8_0", None, [ctypes.POINTER(MatmulParams), _vp, _vp, _vp])
_topk = _sig("bpo_topk_reduce", None, [ctypes.POINTER(TopKParams), _vp, _vp])
_f16_add = _sig("bpo_f16_add", ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint16])
_f16_mul = _sig("bpo_f16_mul", ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint16])
_mv = _sig("bpo_matvec_q1_0", None, [ctypes.POINTER(MatvecParams), _vp, _vp])
_mv_silu = _sig("bpo_matvec_q1_0_silu", None, [ctypes.POINTER(MatvecSiluParams), _vp, _vp])
_mv_normed = _sig("bpo_matvec_q1_0_fused_normed", None, [ctypes.POINTER(MatvecFusedNormedParams), _vp,
                                                         _vp, _vp])


def _ptr(a):
    return a.ctypes.data_as(_vp) if a is not None else None


def _u16(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16) if a.dtype == np.float16 else a


# ---- conversions -------------------------------------------------------------
def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    _f32_to_f16_arr(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    _f16_to_f32_arr(_ptr(h), _ptr(out), h.size)
    return out


# ---- tables / layout -----------------------------------------------------------
def rope_table(head_dim: int, base: float, max_seq: int):
    """(f32 table, f16-bit table), each [max_seq * head_dim]."""
    f = np.empty(max_seq * head_dim, np.float32)
    h = np.empty(max_seq * head_dim, np.uint16)
    _rope(head_dim, base, max_seq, _ptr(f), _ptr(h))
    return f, h


def kv_layer_offsets(n_layer, kv_dim, max_seq, il):
    d, q = _u64(), _u64()
    _layer_off(n_layer, kv_dim, max_seq, il, ctypes.byref(d), ctypes.byref(q))
    return d.value, q.value


def kv_buffer_bytes(n_layer, kv_dim, max_seq):
    return _buf_bytes(n_layer, kv_dim, max_seq)


def snapshot_payload_bytes(n_layer, kv_dim, pos):
    return _snap_bytes(n_layer, kv_dim, pos)


def snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, sect):
    return _snap_off(n_layer, kv_dim, pos, kind, il, sect)


def snapshot_capture(n_layer, kv_dim, max_seq, pos, kv_k, kv_v) -> np.ndarray:
    out = np.empty(snapshot_payload_bytes(n_layer, kv_dim, pos), np.uint8)
    _snap_cap(n_layer, kv_dim, max_seq, pos, _ptr(kv_k), _ptr(kv_v), _ptr(out))
    return out


def snapshot_apply(n_layer, kv_dim, max_seq, pos, payload, kv_k, kv_v) -> None:
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    _snap_apply(n_layer, kv_dim, max_seq, pos, _ptr(payload), _ptr(kv_k), _ptr(kv_v))


def quantize_block(x):
    """Q8_0 one block of 32 f32 values -> (d, int8[32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape == (32,)
    d = np.zeros(1, np.float32)
    q = np.zeros(32, np.int8)
    _quant(_ptr(x), _ptr(d), _ptr(q))
    return float(d[0]), q


# ---- kernels ---------------------------------------------------------------------
def kv_writeback_fused(p: KvWritebackParams, act, w_norms, rope_cs, kv_k, kv_v, n_kv_head,
                       m_tokens) -> None:
    """In place on kv_k / kv_v (uint8 arrays)."""
    act, w_norms, rope_cs = _u16(act), _u16(w_norms), _u16(rope_cs)
    assert kv_k.dtype == np.uint8 and kv_v.dtype == np.uint8
    _kvwb(ctypes.byref(p), _ptr(act), _ptr(w_norms), _ptr(rope_cs), _ptr(kv_k), _ptr(kv_v),
          n_kv_head, m_tokens)


def q_norm_rope_fused(p: QNormRopeParams, act, w_norms, rope_cs, n_head, m_tokens) -> None:
    """In place on act (uint16 array)."""
    assert act.dtype == np.uint16 and act.flags.c_contiguous
    w_norms, rope_cs = _u16(w_norms), _u16(rope_cs)
    _qnr(ctypes.byref(p), _ptr(act), _ptr(w_norms), _ptr(rope_cs), n_head, m_tokens)


def attention_split_merge(p: AttnSplitParams, act, kv_k, kv_v):
    """Returns (f16-bit output [n_head*head_dim], f32 output)."""
    act = _u16(act)
    out16 = act.copy()
    out32 = np.empty(p.n_head * p.head_dim, np.float32)
    _split(ctypes.byref(p), _ptr(act), _ptr(kv_k), _ptr(kv_v), _ptr(out16), _ptr(out32))
    o = p.out_offset
    return out16[o:o + p.n_head * p.head_dim].copy(), out32


def attention(p: AttnParams, act, kv_k, kv_v, tokens=None):
    """f32 outputs [n_tokens, n_head*head_dim] for the selected tokens (all if None)."""
    act = _u16(act)
    if tokens is None:
        n = p.m_tokens
        tok = None
    else:
        tok = np.ascontiguousarray(tokens, dtype=np.uint32)
        n = tok.size
    out32 = np.empty((n, p.n_head * p.head_dim), np.float32)
    _attn(ctypes.byref(p), _ptr(act), _ptr(kv_k), _ptr(kv_v), _ptr(tok), n, None, _ptr(out32))
    return out32


def fill_normal_f16(seed: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    _fill(seed, mean, std, _ptr(out), n)
    return out


# ---- Q1_0 matvecs (matvec_q1_0*.wgsl) -----------------------------------------
def f16_add(a: int, b: int) -> int:
    return int(_f16_add(a, b))


def f16_mul(a: int, b: int) -> int:
    return int(_f16_mul(a, b))


def matvec_q1_0(p: MatvecParams, weights: np.ndarray, act) -> np.ndarray:
    """Returns a copy of act (uint16) with the output rows written."""
    out = _u16(act).copy()
    _mv(ctypes.byref(p), _ptr(np.ascontiguousarray(weights, np.uint8)), _ptr(out))
    return out


def matvec_q1_0_silu(p: MatvecSiluParams, weights: np.ndarray, act) -> np.ndarray:
    out = _u16(act).copy()
    _mv_silu(ctypes.byref(p), _ptr(np.ascontiguousarray(weights, np.uint8)), _ptr(out))
    return out


def matvec_q1_0_fused_normed(p: MatvecFusedNormedParams, weights: np.ndarray, act, w_norms) -> np.ndarray:
    out = _u16(act).copy()
    _mv_normed(ctypes.byref(p), _ptr(np.ascontiguousarray(weights, np.uint8)), _ptr(out),
               _ptr(_u16(w_norms)))
    return out


def q1_0_tensor(rng: np.random.Generator, n: int, k: int, d_scale=0.02):
    """Random Q1_0 tensor (d f16 then qs, the model.rs:784-804 layout) as bytes,
    with the d / qs byte offsets relative to its start."""
    nb = k // 128
    d = (rng.standard_normal(n * nb) * d_scale).astype(np.float16)
    qs = rng.integers(0, 256, size=n * nb * 16, dtype=np.uint8)
    d_bytes = d.view(np.uint8)
    qs_off = (d_bytes.size + 3) // 4 * 4
    buf = np.zeros(qs_off + qs.size, np.uint8)
    buf[:d_bytes.size] = d_bytes
    buf[qs_off:] = qs
    return buf, 0, qs_off


# ---- prefill projections (quantize_q8_0.wgsl, matmul_q1_0_q8_0.wgsl) ---------
def quantize_act_q8_0(p: QuantParams, act, outbuf: np.ndarray) -> np.ndarray:
    """Returns a copy of outbuf (uint8) with the Q8_0 d / qs regions written."""
    out = np.ascontiguousarray(outbuf, np.uint8).copy()
    _quant_act(ctypes.byref(p), _ptr(_u16(act)), _ptr(out))
    return out


def matmul_q1_0_q8_0(p: MatmulParams, weights: np.ndarray, acts: np.ndarray, y) -> np.ndarray:
    """Returns a copy of y (uint16, the f16 activation buffer) with the output written."""
    out = _u16(y).copy()
    _matmul(ctypes.byref(p), _ptr(np.ascontiguousarray(weights, np.uint8)),
            _ptr(np.ascontiguousarray(acts, np.uint8)), _ptr(out))
    return out


def topk_reduce(p: "TopKParams", act, result) -> np.ndarray:
    """Returns a copy of result (uint32 words) with the top-k values (f32 bits,
    descending) and their indices written at p.out_offset."""
    out = np.ascontiguousarray(result, np.uint32).copy()
    _topk(ctypes.byref(p), _ptr(_u16(act)), _ptr(out))
    return out
