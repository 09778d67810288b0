"""BONSAIKV v1 KV-cache snapshots, byte-compatible with the reference's
``KvSnapshot`` (src/kv_snapshot.rs in the reference repository).

Blob = 32-byte header (magic "BONSAIKV", u32 LE version=1, n_layer, kv_dim,
max_seq, pos, reserved=0; src/kv_snapshot.rs:66-80) + payload ordered
for kind in {K, V}: for each layer: d-section (pos*(kv_dim/32)*4 bytes of
FP32 scales) then qs-section (pos*kv_dim bytes of i8) (:8-17).
"""
import struct
from dataclasses import dataclass

from .errors import ConfigError, ContextOverflowError
from .layout import snapshot_payload_bytes

MAGIC = b"BONSAIKV"
VERSION = 1
HEADER_BYTES = 32


@dataclass
class KvSnapshot:
    n_layer: int
    kv_dim: int
    max_seq: int
    pos: int
    payload: bytes

    def to_bytes(self) -> bytes:
        """src/kv_snapshot.rs:66-80."""
        hdr = MAGIC + struct.pack("<6I", VERSION, self.n_layer, self.kv_dim, self.max_seq,
                                  self.pos, 0)
        return hdr + bytes(self.payload)

    @classmethod
    def from_bytes(cls, blob: bytes) -> "KvSnapshot":
        """src/kv_snapshot.rs:99-140: same checks, same order."""
        if len(blob) < HEADER_BYTES:
            raise ConfigError("KvSnapshot blob too short: missing header")
        if blob[0:8] != MAGIC:
            raise ConfigError("KvSnapshot blob has wrong magic")
        version, n_layer, kv_dim, max_seq, pos, reserved = struct.unpack("<6I", blob[8:32])
        if version != VERSION:
            raise ConfigError("KvSnapshot blob has unsupported version")
        if reserved != 0:
            raise ConfigError("KvSnapshot blob has non-zero reserved field")
        if len(blob) - HEADER_BYTES != snapshot_payload_bytes(n_layer, kv_dim, pos):
            raise ConfigError("KvSnapshot blob payload length does not match header")
        return cls(n_layer, kv_dim, max_seq, pos, bytes(blob[HEADER_BYTES:]))

    # -- GPU paths (src/kv_snapshot.rs:203-372) -------------------------------------
    @classmethod
    def capture(cls, model, pos: int) -> "KvSnapshot":
        cfg = model.cfg
        payload = model.snapshot_payload(pos) if pos else b""
        return cls(cfg.n_layer, cfg.kv_dim, model.max_seq, pos, payload)

    def validate_against(self, model) -> None:
        """src/kv_snapshot.rs:184-198."""
        if self.n_layer != model.cfg.n_layer or self.kv_dim != model.cfg.kv_dim:
            raise ConfigError("KvSnapshot does not match model: n_layer or kv_dim differs")
        if self.pos > model.max_seq:
            raise ContextOverflowError(
                f"context overflow: pos 0 + tokens {self.pos} > max_seq {model.max_seq}")

    def apply(self, model) -> None:
        self.validate_against(model)
        if self.pos == 0:
            return
        model.apply_payload(self.pos, self.payload)
