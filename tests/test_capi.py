"""CPU-side tests of the C ABI library and the host mirror: the library loads,
exports every symbol include/bonsai_pot_hip.h declares, its host-only helpers
agree with the layout restatements, config validation and error mapping
behave like the reference's, and KvSnapshot blobs follow BONSAIKV v1
(the reference's src/kv_snapshot.rs tests)."""
import ctypes
import os
import re
import struct

import pytest

import bonsai_pot_amd as bp
from bonsai_pot_amd import errors, layout
from bonsai_pot_amd.snapshot import HEADER_BYTES, KvSnapshot

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bonsai_pot_hip.h")


BENCH_HEADER = os.path.join(ROOT, "include", "bonsai_pot_hip_bench.h")


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(bp.lib, n), f"{n} declared in include/ but not exported"
    assert set(names) == set(bp.EXPORTED_SYMBOLS)


def test_bench_hooks_only_in_bench_build():
    """The measurement hooks (include/bonsai_pot_hip_bench.h) are exported by
    the bench build of the library and not by the product library."""
    names = declared_functions(BENCH_HEADER)
    assert set(names) == set(bp.model.BENCH_SYMBOLS)
    product = ctypes.CDLL(os.path.join(os.path.dirname(bp.library_path), "libbonsai_pot_hip.so"))
    bench = ctypes.CDLL(os.path.join(os.path.dirname(bp.library_path), "libbonsai_pot_hip_bench.so"))
    for n in names:
        assert not hasattr(product, n), f"{n} exported by the product library"
        assert hasattr(bench, n), f"{n} missing from the bench build"
    for n in declared_functions():
        assert hasattr(bench, n), f"{n} missing from the bench build"


def test_library_is_gfx950_hip_build():
    data = open(bp.library_path, "rb").read()
    assert b"gfx950" in data
    assert b"amdgcn-amd-amdhsa" in data


def test_host_helpers_match_layout():
    for n_layer, max_seq, il in [(36, 32768, 35), (1, 513, 0), (36, 4097, 17)]:
        d, q = ctypes.c_uint64(), ctypes.c_uint64()
        assert bp.lib.bp_kv_layer_offsets(n_layer, 1024, max_seq, il, ctypes.byref(d), ctypes.byref(q)) == 0
        assert (d.value, q.value) == layout.kv_layer_offsets(n_layer, 1024, max_seq, il)
        assert bp.lib.bp_kv_buffer_bytes(n_layer, 1024, max_seq) == layout.kv_buffer_bytes(n_layer, 1024, max_seq)
    assert bp.lib.bp_kv_snapshot_payload_bytes(36, 1024, 512) == 42_467_328
    assert bp.lib.bp_kv_snapshot_payload_bytes(36, 1024, 32768) == 2_717_908_992
    d = ctypes.c_uint64()
    assert bp.lib.bp_kv_layer_offsets(36, 1024, 1024, 36, ctypes.byref(d), None) == errors.BP_ERR_INVALID_ARG


def test_status_names():
    assert bp.lib.bp_status_name(0) == b"BP_OK"
    assert bp.lib.bp_status_name(-5) == b"BP_ERR_DEVICE_LOST"
    assert bp.lib.bp_status_name(-99) == b"BP_ERR_UNKNOWN"


def test_config_validation_before_device():
    # src/model.rs:1179-1183: head_dim must be 128 -> PotError::Config
    with pytest.raises(bp.ConfigError, match="head_dim"):
        bp.Model(layout.Config(head_dim=64), 128)
    with pytest.raises(bp.ConfigError, match="n_head"):
        bp.Model(layout.Config(n_head=16), 128)
    with pytest.raises(bp.ConfigError):
        bp.Model(layout.Config(), 0)


def test_max_seq_guard_for_32bit_layer_offsets():
    # The kernels address rows inside one layer with 32-bit offsets
    # (row * kv_dim + column), so max_seq * kv_dim must fit in 2^32; the check
    # runs before any device query, so it is a Config error on any host.
    kv_dim = 1024
    limit = (1 << 32) // kv_dim          # 4,194,304 rows: exactly 2^32 bytes per layer
    with pytest.raises(bp.ConfigError, match="32-bit"):
        bp.Model(layout.Config(n_layer=1), limit + 1)
    with pytest.raises(bp.ConfigError, match="32-bit"):
        bp.Model(layout.Config(n_layer=1, n_head=64, n_kv_head=16), limit // 2 + 1)


def test_no_device_maps_to_no_adapter():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    with pytest.raises(bp.NoAdapterError):
        bp.Model(layout.Config(n_layer=1), 128)


def test_null_model_is_invalid_arg():
    assert bp.lib.bp_check_device(None) == errors.BP_ERR_INVALID_ARG
    assert b"NULL" in bp.lib.bp_last_error()
    assert bp.lib.bp_dispatch_attention(None, None, 0, 0, 0, 0, 1, 1) == errors.BP_ERR_INVALID_ARG
    assert bp.lib.bp_dispatch_attention_prefill_step(None, None, None, 0, 0, 0, 0, 0, 0, 0, 0, 1) == \
        errors.BP_ERR_INVALID_ARG


# ---- KvSnapshot blob (src/kv_snapshot.rs:376-521) ----------------------------------
def make_snap(n_layer, kv_dim, max_seq, pos):
    n = layout.snapshot_payload_bytes(n_layer, kv_dim, pos)
    return KvSnapshot(n_layer, kv_dim, max_seq, pos, bytes(i & 0xFF for i in range(n)))


def test_snapshot_header_roundtrip():
    s = make_snap(36, 1024, 1024, 4)
    b = s.to_bytes()
    assert b[:8] == b"BONSAIKV" and struct.unpack("<6I", b[8:32]) == (1, 36, 1024, 1024, 4, 0)
    s2 = KvSnapshot.from_bytes(b)
    assert (s2.n_layer, s2.kv_dim, s2.max_seq, s2.pos, s2.payload) == \
        (36, 1024, 1024, 4, s.payload)


def test_snapshot_empty_roundtrip():
    s = make_snap(36, 1024, 1024, 0)
    b = s.to_bytes()
    assert len(b) == HEADER_BYTES
    assert KvSnapshot.from_bytes(b).pos == 0


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"\xff" + b[1:], "magic"),
    (lambda b: b[:8] + struct.pack("<I", 2) + b[12:], "version"),
    (lambda b: b[:28] + struct.pack("<I", 1) + b[32:], "reserved"),
    (lambda b: b[:-1], "payload length"),
    (lambda b: b[:31], "too short"),
])
def test_snapshot_from_bytes_rejects(mutate, msg):
    b = make_snap(36, 1024, 1024, 4).to_bytes()
    with pytest.raises(bp.ConfigError, match=msg):
        KvSnapshot.from_bytes(mutate(b))


def test_snapshot_validate_against_model_shape():
    class FakeModel:
        cfg = layout.Config(n_layer=36)
        max_seq = 8
    make_snap(36, 1024, 1024, 8).validate_against(FakeModel)
    with pytest.raises(bp.ContextOverflowError):
        make_snap(36, 1024, 1024, 9).validate_against(FakeModel)
    with pytest.raises(bp.ConfigError):
        make_snap(35, 1024, 1024, 4).validate_against(FakeModel)
