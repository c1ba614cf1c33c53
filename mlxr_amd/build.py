"""Build libmlxr_qgemm.so (HIP, gfx950) in-tree with hipcc, and beside it libmlxr_bench.so
(the benchmark's measurement probes, kept out of the matmul library).

Objects go to mlxr_amd/_build/, the libraries to mlxr_amd/lib/.  Every call recompiles.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libmlxr_qgemm.so")
BENCH_LIB = os.path.join(LIBDIR, "libmlxr_bench.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# longest compiles first (the pool starts them first)
SOURCES = ["qgemm_gemv.hip", "qgemm_mlp.hip", "qgemm_tile_q4k.hip", "qgemm_tile_q6k.hip", "qgemm_tile_q5k.hip",
           "qgemm_tile_q40.hip", "qgemm_tile_q41.hip", "qgemm_tile_q80.hip", "qgemm_skinny.hip",
           "qgemm_tile.hip", "qgemm_api.hip", "qgemm_pack.hip", "qgemm_noalloc.hip",
           "q_gemm_dequant_primitive.cpp", "synth.cpp", "gguf.cpp", "act.hip", "linear.cpp"]
BENCH_SOURCES = ["bench_probe.hip"]
COMMON = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-Wall",
          # packed fp32 VALU ops are kept out of the device code
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", os.path.join(HERE, "..", "include")]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + COMMON + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{errs}")
    return obj, errs


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        results = list(ex.map(_compile, SOURCES + BENCH_SOURCES))
    for _, msg in results:
        if msg.strip() and verbose:
            print(msg, file=sys.stderr)
    objs = [o for o, _ in results]
    nb = len(BENCH_SOURCES)
    for lib, part in ((LIB, objs[:-nb]), (BENCH_LIB, objs[-nb:])):
        cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", lib] + part
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
