"""Python binding of the MI355X attention hot path of bonsai-pot.

This is a thin ctypes layer over ``lib/libbonsai_pot_hip.so`` (the C ABI in
``include/bonsai_pot_hip.h``), shaped like the reference's Rust host side
(paths relative to the reference repository root):

* :class:`Model` — the attention part of ``Model`` (src/model.rs): owns the
  Q8_0 ``kv_k``/``kv_v`` cache, the f16 RoPE table and the split-K scratch;
  its ``dispatch_*`` methods are the dispatch helpers of src/forward.rs.
* :class:`KvSnapshot` — ``KvSnapshot`` (src/kv_snapshot.rs), the BONSAIKV v1
  blob, byte-compatible with the reference.
* :class:`PotError` and subclasses — ``PotError`` (src/error.rs).

All device arguments are raw device addresses (ints), e.g. a torch tensor's
``data_ptr()``. There is no CPU fallback: importing raises if the HIP library
has not been built.
"""
from .errors import (PotError, ConfigError, ContextOverflowError, DeviceLostError,
                     HipError, NoAdapterError, OutOfMemoryError)
from .layout import (Config, BONSAI_4B, BONSAI_8B, kv_layer_offsets, kv_buffer_bytes,
                     snapshot_payload_bytes, snapshot_payload_offset)
from .model import Model, lib, library_path, EXPORTED_SYMBOLS
from .snapshot import KvSnapshot

__all__ = [
    "PotError", "ConfigError", "ContextOverflowError", "DeviceLostError", "HipError",
    "NoAdapterError", "OutOfMemoryError", "Config", "BONSAI_4B", "BONSAI_8B",
    "kv_layer_offsets", "kv_buffer_bytes", "snapshot_payload_bytes",
    "snapshot_payload_offset", "Model", "KvSnapshot", "lib", "library_path",
    "EXPORTED_SYMBOLS",
]
