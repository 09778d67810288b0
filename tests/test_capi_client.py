"""A compiled C program as the ABI's caller (tests/capi_client.c): it includes
only include/bonsai_pot_hip.h (and the HIP runtime API for its own device
buffers) and links libbonsai_pot_hip.so, as the reference-side -sys crate
would. CPU: the header is self-sufficient C99 and the program links against
the library; without a device the program reports BP_ERR_NO_DEVICE through
the ABI's own error strings. GPU: one decode step of configs[1]'s shape,
both as the reference's three dispatches and as the fused entry point, run by
the C program and compared with the oracle (cache bytes bit-exact, attention
within the tolerance)."""
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

import bonsai_pot_amd as bp
from bonsai_pot_amd import layout
from helpers import Scenario, assert_attn_close

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "capi_client.c")
LIBDIR = os.path.dirname(bp.library_path)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build_client(out_dir) -> str:
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = os.path.join(str(out_dir), "capi_client")
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROCM, "include"), "-D__HIP_PLATFORM_AMD__", SRC, "-o", exe,
           "-L", LIBDIR, "-lbonsai_pot_hip", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
           f"-Wl,-rpath,{LIBDIR}", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return exe


def test_header_is_self_sufficient_c(tmp_path):
    """The public header compiles on its own as C99 and C++ with warnings as errors."""
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    for lang, std, comp in (("c", "-std=c99", "gcc"), ("c++", "-std=c++17", "g++")):
        src = tmp_path / f"only_header.{ 'c' if lang == 'c' else 'cpp'}"
        src.write_text('#include "bonsai_pot_hip.h"\nint main(void) { return bp_status_name(BP_OK) == 0; }\n')
        r = subprocess.run([comp, std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-I",
                            os.path.join(ROOT, "include"), "-c", str(src), "-o", str(tmp_path / f"o_{lang}.o")],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr


def test_client_links_and_reports_no_device(tmp_path):
    import torch
    exe = build_client(tmp_path)
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present (the GPU test runs the client)")
    inp = tmp_path / "in.bin"
    inp.write_bytes(struct.pack("<6I", 1, 16, 0, 0, 0, 0) + bytes(2 * layout.kv_buffer_bytes(1, 1024, 16)))
    r = subprocess.run([exe, str(inp), str(tmp_path / "out.bin")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2, r.stdout + r.stderr
    assert "BP_ERR_NO_DEVICE" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("pos", [0, 700])
def test_client_decode_step_matches_oracle(cuda, tmp_path, pos):
    print(f"[capi_client] decode step pos={pos}", flush=True)
    sys.stdout.flush()
    exe = build_client(tmp_path)
    cfg = layout.Config(n_layer=3)
    max_seq, il = 768, 2
    sc = Scenario(cfg, max_seq=max_seq, m_tokens=1, seed=900 + pos, w_std=0.1)
    assert (sc.q_off, sc.k_off, sc.v_off, sc.out_off) == (0, 4096, 5120, 6144)
    assert (sc.w_q_off, sc.w_k_off) == (0, 128)
    if pos:
        pre = Scenario(cfg, max_seq, pos, seed=901 + pos, with_q=False)
        pre.oracle_writeback(il, 0)
        sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    inp = tmp_path / "in.bin"
    with open(inp, "wb") as f:
        f.write(struct.pack("<6I", cfg.n_layer, max_seq, il, pos, sc.act.size, sc.w_norms.size))
        f.write(sc.act.tobytes())
        f.write(sc.w_norms.tobytes())
        f.write(sc.kv_k.tobytes())
        f.write(sc.kv_v.tobytes())
    outp = tmp_path / "out.bin"
    r = subprocess.run([exe, str(inp), str(outp)], capture_output=True, text=True, timeout=120)
    print(r.stdout + r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(il, pos)
    _, want = sc.oracle_decode(il, pos)
    raw = np.fromfile(outp, np.uint8)
    n_act, nkv = 2 * sc.act.size, sc.kv_k.size
    assert raw.size == 2 * (n_act + 2 * nkv)
    for run in range(2):
        base = run * (n_act + 2 * nkv)
        act = raw[base:base + n_act].view(np.uint16)
        k = raw[base + n_act:base + n_act + nkv]
        v = raw[base + n_act + nkv:base + n_act + 2 * nkv]
        tag = ["three dispatches", "fused step"][run]
        assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), f"{tag}: cache bytes differ"
        assert np.array_equal(act[:4096], sc.act[:4096]), f"{tag}: normalized q differs"
        got = act[sc.out_off:sc.out_off + 4096].view(np.float16).astype(np.float32)
        err = assert_attn_close(got, want, f"C client {tag} pos {pos}")
        print(f"[capi_client] {tag} pos={pos}: max_abs {err[0]:.2e} rel_l2 {err[1]:.2e}", flush=True)
