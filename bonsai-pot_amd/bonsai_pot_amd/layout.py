"""Model shapes and the Q8_0 KV-cache / snapshot byte layout.

Pure-Python restatement of the reference's layout helpers (paths relative to
the reference repository root), used by callers to size and address buffers:

* ``kv_layer_offsets``        src/forward.rs:48-58
* ``kv_buffer_bytes``         src/model.rs:1184-1187
* ``snapshot_payload_*``      src/kv_snapshot.rs:145-169
"""
from dataclasses import dataclass


@dataclass(frozen=True)
class Config:
    """Attention-side subset of ``Config`` (src/model.rs:568-656)."""
    n_layer: int = 36
    n_head: int = 32
    n_kv_head: int = 8
    head_dim: int = 128
    rms_eps: float = 1e-6
    rope_freq_base: float = 1e6

    @property
    def kv_dim(self) -> int:
        return self.n_kv_head * self.head_dim

    @property
    def q_dim(self) -> int:
        return self.n_head * self.head_dim


# Bonsai 4B and 8B have identical attention shapes (src/kv_snapshot.rs:437-441).
BONSAI_4B = Config()
BONSAI_8B = Config()


def kv_qs_byte_base(n_layer: int, kv_dim: int, max_seq: int) -> int:
    return n_layer * max_seq * (kv_dim // 32) * 4


def kv_layer_offsets(n_layer: int, kv_dim: int, max_seq: int, il: int):
    """(u32-word offset of layer il's d-section, byte offset of its qs-section)."""
    d_word = il * max_seq * (kv_dim // 32)
    qs_byte = kv_qs_byte_base(n_layer, kv_dim, max_seq) + il * max_seq * kv_dim
    return d_word, qs_byte


def kv_buffer_bytes(n_layer: int, kv_dim: int, max_seq: int) -> int:
    return n_layer * max_seq * (kv_dim // 32) * 4 + n_layer * max_seq * kv_dim


def snapshot_payload_bytes(n_layer: int, kv_dim: int, pos: int) -> int:
    d_layer = pos * (kv_dim // 32) * 4
    qs_layer = pos * kv_dim
    return 2 * n_layer * (d_layer + qs_layer)


def snapshot_payload_offset(n_layer: int, kv_dim: int, pos: int, kind: int, il: int,
                            sect: int) -> int:
    """kind 0 = K, 1 = V; sect 0 = d (FP32 scales), 1 = qs (i8 quants)."""
    d_layer = pos * (kv_dim // 32) * 4
    qs_layer = pos * kv_dim
    layer_bytes = d_layer + qs_layer
    base = kind * n_layer * layer_bytes + il * layer_bytes
    return base if sect == 0 else base + d_layer
