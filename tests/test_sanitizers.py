"""AddressSanitizer / UndefinedBehaviorSanitizer runs of the CPU-side code.

1. The C oracle (oracle/bp_oracle.c) is rebuilt with
   -fsanitize=address,undefined (`make -C oracle asan`) and the oracle's own
   CPU test files are run against that build in a child process with the ASan
   runtime preloaded into the interpreter. Every out-of-bounds read or write
   of an oracle routine on the arrays the tests hand it (numpy allocations go
   through the intercepted malloc) and every UB report aborts the child.
2. A negative control shows the sanitizer is live in that configuration: a
   deliberately short output array handed to the Q8_0 block quantizer through
   ctypes must be reported as a heap-buffer-overflow.
3. The C-ABI client program (tests/capi_client.c) is built with
   -fsanitize=address,undefined and run on the no-device path of the library.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")
ASAN_LIB = os.path.join(ORACLE, "_asan", "libbp_oracle.so")


def _runtime():
    if shutil.which("gcc") is None or shutil.which("make") is None:
        pytest.skip("gcc/make not available")
    rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(rt) or not os.path.exists(rt):
        pytest.skip("libasan runtime not found")
    return rt


@pytest.fixture(scope="module")
def asan_env():
    rt = _runtime()
    r = subprocess.run(["make", "-s", "-C", ORACLE, "asan"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ)
    env.update(BP_ORACLE_LIB=ASAN_LIB, LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:exitcode=87")
    return env


def test_oracle_tests_under_asan_ubsan(asan_env):
    files = ["test_oracle.py", "test_golden.py", "test_topk_wgsl_sim.py", "test_matmul.py", "test_topk.py",
             "test_matvec.py"]
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider"]
    cmd += [os.path.join(ROOT, "tests", f) for f in files]
    r = subprocess.run(cmd, cwd=ROOT, env=asan_env, capture_output=True, text=True, timeout=900)
    out = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, out
    assert "passed" in r.stdout, out


def test_sanitizer_is_live(asan_env):
    """An oracle call with a 16-byte output where 32 are written must be caught."""
    prog = (
        "import sys, ctypes, numpy as np\n"
        f"sys.path.insert(0, {ORACLE!r})\n"
        "import oracle as orc\n"
        f"assert orc.LIB_PATH == {ASAN_LIB!r}\n"
        "x = np.linspace(-1, 1, 32).astype(np.float32)\n"
        "d = np.zeros(1, np.float32); q = np.zeros(16, np.int8)\n"
        "orc._quant(orc._ptr(x), orc._ptr(d), orc._ptr(q))\n"
        "print('not caught')\n")
    r = subprocess.run([sys.executable, "-c", prog], env=asan_env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 86, r.stdout + r.stderr
    assert "heap-buffer-overflow" in r.stderr
    assert "not caught" not in r.stdout


def test_capi_client_no_device_under_asan(tmp_path):
    """The C client program, built with ASan+UBSan, on the library's no-device path."""
    import struct

    import torch

    _runtime()
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present (this covers the no-device path)")
    import bonsai_pot_amd as bp
    from bonsai_pot_amd import layout
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    libdir = os.path.dirname(bp.library_path)
    exe = str(tmp_path / "capi_client_asan")
    cmd = ["gcc", "-std=c99", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(rocm, "include"), "-D__HIP_PLATFORM_AMD__",
           os.path.join(ROOT, "tests", "capi_client.c"), "-o", exe, "-L", libdir, "-lbonsai_pot_hip",
           "-L", os.path.join(rocm, "lib"), "-lamdhip64", f"-Wl,-rpath,{libdir}",
           f"-Wl,-rpath,{os.path.join(rocm, 'lib')}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    inp = tmp_path / "in.bin"
    inp.write_bytes(struct.pack("<6I", 1, 16, 0, 0, 0, 0) + bytes(2 * layout.kv_buffer_bytes(1, 1024, 16)))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:exitcode=86")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe, str(inp), str(tmp_path / "out.bin")], capture_output=True, text=True, timeout=120,
                       env=env)
    assert r.returncode == 2, r.stdout + r.stderr
    assert "BP_ERR_NO_DEVICE" in r.stderr
