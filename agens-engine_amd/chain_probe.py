"""Per-step phase times of the chained M = 1 sweep (a measurement tool, not part of the library).

A probe build of libagens_kernels.so (wq_i8m1d.hip compiled with -DAK_CHAIN_PROBE) records, per chained step and
workgroup, wall-clock marks at the step's start, its activations ready (wave 0), converted (all waves), its item loop
done, its outputs issued and its closing barrier; this tool builds that library beside the package (in _probe/) and
runs the benchmark sweep of bench.py through it, then prints per step class (mean over the sweep's steps of that class):
the step's span (from the last output of the step before to its own last output), when its workgroups have their
activations after the step before's last output (first / median / last workgroup), the conversion, the item loop
(mean / max over workgroups), the output phase, and the straggler tail (last workgroup's outputs minus the median's).

  python agens-engine_amd/chain_probe.py --build        # on the build host, after `python agens-engine_amd/build.py`
  python agens-engine_amd/chain_probe.py [--m 1] [--tp 1] [--npy out.npy]    # on an MI355X
"""
import argparse
import collections
import ctypes
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PROBE = os.path.join(HERE, "_probe")
SLOTS = 6        # marks per (step, workgroup): start, x ready, converted, loop done, outputs issued, step end
RING = 1024      # steps of the record ring (indexed by the step's flag target mod RING)
WGS = 256


def build():
    sys.path.insert(0, HERE)
    import build as B  # the package's build script: flags, sources, object directory
    os.makedirs(PROBE, exist_ok=True)
    obj = os.path.join(PROBE, "wq_i8m1d.o")
    cmd = [B.hipcc()] + B.flags() + ["-DAK_CHAIN_PROBE", "-c", os.path.join(B.CSRC, "wq_i8m1d.hip"), "-o", obj]
    subprocess.run(cmd, check=True, capture_output=True)
    objs = [os.path.join(B.BUILD, os.path.splitext(s)[0] + ".o") for s in B.SOURCES if s != "wq_i8m1d.hip"]
    missing = [o for o in objs if not os.path.exists(o)]
    if missing:
        raise SystemExit(f"{missing[0]} missing: run `python agens-engine_amd/build.py` first")
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    lib = os.path.join(PROBE, "libagens_kernels.so")
    subprocess.run([B.hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", lib] + objs +
                   [obj, "-L" + rocm_lib, "-lrocblas", "-Wl,-rpath," + rocm_lib], check=True)
    subprocess.run([B.hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o",
                    os.path.join(PROBE, "libagens_bench.so"), os.path.join(B.BUILD, "bench_support.o"), "-L" + PROBE,
                    "-lagens_kernels", "-Wl,-rpath,$ORIGIN"], check=True)
    os.remove(obj)
    print(f"built {lib}")


def record(m, tp):
    """Runs the sweep chained (3 untimed runs, then the recorded one) and returns the marks [step][wg][SLOTS] in
    wall-clock ticks (100 MHz) and the steps' (class, bits)."""
    sys.path.insert(0, ROOT)
    import bench
    bench.PKG = PROBE
    K, B = bench.load_libs()
    K.ak_chain_probe_read.restype = ctypes.c_int
    K.ak_chain_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint32)]
    ctx = bench.Ctx(K, B)
    plan, meta, _ = bench.build_sweep(ctx, m, 0, tp)
    arr = (bench.AgbLaunch * len(plan))(*plan)
    ms, chained, status = ctypes.c_float(), ctypes.c_int(), ctypes.c_int()
    ctx.check(B.agb_run_chain(arr, len(plan), 3, 1, 0, ctypes.byref(ms), ctypes.byref(chained),
                              ctypes.byref(status)), "chained run")
    if chained.value != 1 or status.value != 0:
        raise SystemExit(f"the sweep did not run as one chained launch (chained {chained.value}, status {status.value})")
    buf = np.zeros(RING * WGS * SLOTS, np.uint64)
    flag0 = ctypes.c_uint32()
    ctx.check(K.ak_chain_probe_read(buf.ctypes.data, buf.nbytes, ctypes.byref(flag0)), "probe read")
    rec = buf.reshape(RING, WGS, SLOTS).astype(np.int64)
    f0 = flag0.value - len(plan)  # the recorded run's first flag target
    marks = np.stack([rec[(f0 + s) % RING] for s in range(len(plan))])
    print(f"# chained sweep (probe build, eager launch): {ms.value * 1e3:.1f} us", flush=True)
    return marks, meta


def summarize(marks, meta):
    us = 0.01  # per wall-clock tick
    rows = collections.defaultdict(list)
    prev_last = None
    for s in range(marks.shape[0]):
        r = marks[s].copy()
        start = r[:, 0]
        r[:, 1] = np.where(r[:, 1] >= start, r[:, 1], start)  # activations read before the weights: no mark
        valid = np.all(r[:, 1:5] >= start[:, None], axis=1)   # workgroups with rows in the step
        v = r[valid]
        last = v[:, 4].max()
        d = {"conversion": np.mean(v[:, 2] - v[:, 1]) * us, "loop mean": np.mean(v[:, 3] - v[:, 2]) * us,
             "loop max": np.max(v[:, 3] - v[:, 2]) * us, "outputs": np.mean(v[:, 4] - v[:, 3]) * us,
             "tail": (last - np.median(v[:, 4])) * us}
        if prev_last is not None:
            d["span"] = (last - prev_last) * us
            for q, name in ((0, "x first"), (50, "x median"), (100, "x last")):
                d[name] = (np.percentile(v[:, 1], q) - prev_last) * us
        prev_last = last
        rows[f"{meta[s][0]} W{meta[s][1]}"].append(d)
    keys = ["span", "x first", "x median", "x last", "conversion", "loop mean", "loop max", "outputs", "tail"]
    print("| step class | steps | " + " | ".join(keys) + " |")
    print("|---|---|" + "---|" * len(keys))
    for name, ds in sorted(rows.items()):
        vals = [np.mean([d[k] for d in ds if k in d]) if any(k in d for d in ds) else float("nan") for k in keys]
        print(f"| {name} | {len(ds)} | " + " | ".join(f"{x:.2f}" for x in vals) + " |")


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--build", action="store_true", help="build the probe library (no GPU needed)")
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--tp", type=int, default=1)
    ap.add_argument("--npy", help="also save the raw marks [step][workgroup][6] (wall-clock ticks) here")
    a = ap.parse_args()
    if a.build:
        build()
        return
    marks, meta = record(a.m, a.tp)
    if a.npy:
        np.save(a.npy, marks)
    summarize(marks, meta)


if __name__ == "__main__":
    main()
