"""Build recipe for the gfx950 shared library libbonsai_pot_hip.so (in-tree).

Every source under csrc/ is compiled by hipcc for gfx950 only, with
-ffp-contract=off (the norm/RoPE/quantize stages are bit-exact by construction
and must not be fused into FMAs behind their back) and with packed-FP32 ops
disabled for device code.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib", "libbonsai_pot_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
SOURCES = ["bp_api.cpp", "norm_rope_writeback.hip", "attn_decode.hip", "attn_prefill.hip", "matvec_q1_0.hip", "matvec_q1_0_mfma.hip", "matmul_q1_0_q8_0.hip", "topk_reduce.hip"]
# The bench build (lib/libbonsai_pot_hip_bench.so, what bench.py loads): the
# same kernel objects, bp_api.cpp compiled with BP_BENCH_HOOKS (the
# measurement entry points of include/bonsai_pot_hip_bench.h) and the
# read-floor kernel. The product library carries neither.
BENCH_LIB = os.path.join(HERE, "lib", "libbonsai_pot_hip_bench.so")
BENCH_SOURCES = {"bp_api_bench.o": ("bp_api.cpp", ["-DBP_BENCH_HOOKS"]), "read_floor.o": ("read_floor.hip", [])}
# Per-source additions: the matmul's MFMA results go straight to VGPRs (the
# default AGPR form costs one v_accvgpr_read per result element in its f32
# epilogue); the decode kernels' leading scalar arguments (up to 14 dwords)
# are preloaded into SGPRs at wave launch instead of fetched by the first
# scalar loads (a kernel built this way also runs where the command processor
# does not preload: its entry code then loads them itself).
EXTRA_FLAGS = {"matmul_q1_0_q8_0.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               "attn_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}
FLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}) on {cmd[-1]}")
    return r


def build(verbose: bool = False) -> str:
    """Compile every kernel and the host layer, link the product library and
    the bench build, return the product library's path."""
    obj_dir = os.path.join(HERE, "lib", "obj")
    os.makedirs(obj_dir, exist_ok=True)
    jobs = []
    for src in SOURCES:
        obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
        jobs.append((obj, [HIPCC, *FLAGS, *EXTRA_FLAGS.get(src, []), "-c", "-o", obj, os.path.join(CSRC, src)]))
    bench_jobs = []
    for obj_name, (src, defs) in BENCH_SOURCES.items():
        obj = os.path.join(obj_dir, obj_name)
        bench_jobs.append((obj, [HIPCC, *FLAGS, *defs, "-c", "-o", obj, os.path.join(CSRC, src)]))
    with ThreadPoolExecutor(max_workers=4) as ex:
        list(ex.map(lambda j: _run(j[1]), jobs + bench_jobs))
    objs = [o for o, _ in jobs]
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB, *objs])
    bench_objs = [o for o in objs if not o.endswith(os.sep + "bp_api.o")] + [o for o, _ in bench_jobs]
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", BENCH_LIB, *bench_objs])
    if verbose:
        print("built", LIB, "and", BENCH_LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
