"""Builds libagens_kernels.so (the C-ABI library of the mixed-bit GEMV path) in-tree with hipcc for gfx950.

Usage: python agens-engine_amd/build.py [--jobs N]
Objects go to agens-engine_amd/_build/, the library to agens-engine_amd/libagens_kernels.so; also builds the benchmark
helper libagens_bench.so, the C++ host side libagens_linear.so and its test program tests/host/test_linear.
"""
import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libagens_kernels.so")
BENCH_LIB = os.path.join(HERE, "libagens_bench.so")
HOST = os.path.join(HERE, "host")
HOST_LIB = os.path.join(HERE, "libagens_linear.so")
SOURCES = ["ak_runtime.hip", "wq_layout.hip", "wq_exact.hip", "wq_i8.hip", "wq_i8m1d.hip", "wq_i8mt.hip", "wq_api.hip",
           "wq_prefill.hip", "wq_gemm.hip", "wq_mm.hip", "i8_gemv.hip", "bf16_gemv_bi.hip", "silu_mul.hip"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def flags():
    return [
        "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option",
        "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
    ]


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(os.path.splitext(src)[0]) + ".o")
    path = src if os.path.isabs(src) else os.path.join(CSRC, src)
    cmd = [hipcc()] + flags() + ["-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{errs}")
    return obj


def build(jobs=None, verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp] + objs + [
        "-L" + rocm_lib, "-lrocblas", "-Wl,-rpath," + rocm_lib]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    # benchmark support (bench.py only; not part of the product ABI), linked against the library
    bobj = _compile(os.path.join(HERE, "bench", "bench_support.hip"))
    tmp = BENCH_LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp, bobj,
           "-L" + HERE, "-lagens_kernels", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed (bench support):\n" + r.stdout + r.stderr)
    os.replace(tmp, BENCH_LIB)
    # the C++ host side (agens_linear: uploads, linear, linear_shared) and its GPU test program
    gxx = shutil.which("g++") or "g++"
    hflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-I" + os.path.join(ROOT, "include"), "-I" + HOST]
    cmd = [gxx] + hflags + ["-shared", "-o", HOST_LIB + ".tmp", os.path.join(HOST, "agens_linear.cpp"),
                            "-L" + HERE, "-lagens_kernels", "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("host library build failed:\n" + r.stdout + r.stderr)
    os.replace(HOST_LIB + ".tmp", HOST_LIB)
    test_src = os.path.join(ROOT, "tests", "host", "test_linear.cpp")
    test_bin = os.path.join(ROOT, "tests", "host", "test_linear")
    cmd = [gxx] + hflags + ["-o", test_bin + ".tmp", test_src, "-L" + HERE, "-lagens_linear", "-lagens_kernels",
                            "-Wl,-rpath," + HERE]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("host test build failed:\n" + r.stdout + r.stderr)
    os.replace(test_bin + ".tmp", test_bin)
    if verbose:
        print(f"built {LIB}, {BENCH_LIB}, {HOST_LIB} and {test_bin}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    try:
        build(a.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
