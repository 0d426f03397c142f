#!/usr/bin/env python3
"""Benchmark of the mixed-bit quantized GEMV path on one MI355X.

Headline metric: effective HBM GB/s (and % of the 8 TB/s peak) and microseconds per 64-layer
32B-shaped decode GEMV sweep at M = 1: per layer QKV (5120 -> 7168 as q/k/v segments of one launch), O (5120 -> 5120),
gate_up (5120 -> 55296) and down (27648 -> 5120), each layer's bit width drawn from a fixed seed (W2 p=.3, W3 p=.5,
W4 p=.2), group 128, plus the W4 LM head (5120 -> 152064).  One "step" = one sweep (257 GEMV steps, each reading the
previous one's place in the decode order), replayed as one hipGraph (the engine runs decode inside captured graphs),
timed two ways: one launch per linear, and one chained launch (ak_wq_chain_run); the faster is the headline, both are
reported.  Weights are generated on the device in the
reference's int4 container and repacked by ak_wq_repack_kt; inputs are resident in HBM before the timed region.

Effective bytes per launch = packed weights + bf16 scales + bf16 x + bf16 y (the algorithmic bytes).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 1] [--config sweep|0|1|2|3|i8|bi|xover|prefill] [--no-cpu] [--eager]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "agens-engine_amd")
HBM_PEAK_GBS = 8000.0
INT8_PEAK_OPS = 5.0e15  # MI355X dense int8 MFMA peak (ops/s); algorithmic 2*M*n*k is counted against it
SEED = 20261201


class AgbLaunch(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int), ("m", ctypes.c_int), ("nseg", ctypes.c_int), ("k", ctypes.c_int),
                ("group", ctypes.c_int), ("bf16w", ctypes.c_int), ("x", ctypes.c_void_p),
                ("wt", ctypes.c_void_p * 4), ("st", ctypes.c_void_p * 4), ("y", ctypes.c_void_p * 4),
                ("n", ctypes.c_int * 4), ("ldy", ctypes.c_int * 4), ("use_ldy", ctypes.c_int), ("pad", ctypes.c_int)]


def load_libs():
    kso = os.path.join(PKG, "libagens_kernels.so")
    bso = os.path.join(PKG, "libagens_bench.so")
    if not (os.path.exists(kso) and os.path.exists(bso)):
        raise SystemExit(f"{kso} / {bso} missing: run `python agens-engine_amd/build.py` first")
    K = ctypes.CDLL(kso)
    B = ctypes.CDLL(bso)
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    for name, res, args in [
        ("ak_malloc", i, [ctypes.POINTER(vp), sz]), ("ak_free", i, [vp]), ("ak_memcpy_d2h", i, [vp, vp, sz]),
        ("ak_synchronize", i, []), ("ak_wq_kt_weight_bytes", sz, [i, i, i]),
        ("ak_w4_kt_scale_bytes", sz, [i, i, i]), ("ak_wq_repack_kt", i, [i, vp, vp, vp, vp, i, i, i, vp]),
        ("ak_device_name", i, [i, ctypes.c_char_p, i]), ("ak_error_string", ctypes.c_char_p, [i]),
    ]:
        f = getattr(K, name)
        f.restype, f.argtypes = res, args
    for name, res, args in [
        ("agb_gen_container", i, [ctypes.c_uint64, i, i, i, i, vp, vp]),
        ("agb_gen_scales", i, [ctypes.c_uint64, sz, ctypes.c_float, ctypes.c_float, vp, vp]),
        ("agb_gen_x", i, [ctypes.c_uint64, sz, ctypes.c_float, vp, vp]),
        ("agb_run", i, [ctypes.POINTER(AgbLaunch), i, i, i, i, ctypes.POINTER(ctypes.c_float)]),
        ("agb_time_each", i, [ctypes.POINTER(AgbLaunch), i, i, ctypes.POINTER(ctypes.c_float)]),
        ("agb_run_chain", i, [ctypes.POINTER(AgbLaunch), i, i, i, i, ctypes.POINTER(ctypes.c_float),
                              ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
        ("agb_read_bw", i, [sz, i, ctypes.POINTER(ctypes.c_float)]),
        ("agb_gen_i8", i, [ctypes.c_uint64, sz, vp, vp]),
        ("agb_gen_f32", i, [ctypes.c_uint64, sz, ctypes.c_float, ctypes.c_float, vp, vp]),
        ("agb_time_i8_gemv", i, [vp, vp, vp, vp, i, i, i, i, i, i, ctypes.POINTER(ctypes.c_float)]),
        ("agb_time_bi_gemv", i, [vp, vp, vp, i, i, i, i, i, i, ctypes.POINTER(ctypes.c_float)]),
    ]:
        f = getattr(B, name)
        f.restype, f.argtypes = res, args
    return K, B


class Ctx:
    def __init__(self, K, B):
        self.K, self.B, self.bufs = K, B, []

    def check(self, rc, what):
        if rc:
            raise RuntimeError(f"{what}: error {rc} ({self.K.ak_error_string(rc).decode()})")

    def alloc(self, nbytes, keep=True):
        p = ctypes.c_void_p()
        self.check(self.K.ak_malloc(ctypes.byref(p), max(int(nbytes), 16)), "ak_malloc")
        if keep:
            self.bufs.append(p)
        return p

    def free(self, p):
        self.K.ak_free(p)

    def free_all(self):
        for p in self.bufs:
            self.K.ak_free(p)
        self.bufs = []


def code_range(bits):
    return -(1 << (bits - 1)), 1 << bits


class QLinear:
    """A quantized linear generated on the device: container (temporary) -> KT via ak_wq_repack_kt."""

    def __init__(self, ctx, seed, n, k, bits, group=128, ct=None, cs=None, keep_container=False):
        K, B = ctx.K, ctx.B
        self.n, self.k, self.bits, self.group, self.seed = n, k, bits, group, seed
        self.wbytes = K.ak_wq_kt_weight_bytes(bits, n, k)
        self.sbytes = K.ak_w4_kt_scale_bytes(n, k, group)
        self.wt = ctx.alloc(self.wbytes)
        self.st = ctx.alloc(self.sbytes)
        own = ct is None
        if own:
            ct = ctx.alloc(n * k // 2, keep=False)
            cs = ctx.alloc(n * k // group * 2, keep=False)
        lo, span = code_range(bits)
        ctx.check(B.agb_gen_container(seed, n, k, lo, span, ct, None), "gen container")
        # scales |N(0,1)| / sqrt(k E[q^2]) (E[q^2] of uniform codes): outputs stay about unit size through the sweep's
        # data flow, each step reading the one before it
        eq2 = {4: 21.5, 3: 5.5, 2: 1.5}[bits]
        ctx.check(B.agb_gen_scales(seed + 1, n * k // group, float(1.0 / np.sqrt(k * eq2)), 1e-6, cs, None),
                  "gen scales")
        ctx.check(K.ak_wq_repack_kt(bits, ct, cs, self.wt, self.st, n, k, group, None), "repack")
        self.container = None
        if keep_container:  # host copy of the container for the CPU baseline
            p = np.zeros(n * k // 8, dtype=np.uint32)
            s = np.zeros(n * k // group, dtype=np.uint16)
            ctx.check(K.ak_synchronize(), "sync")
            ctx.check(K.ak_memcpy_d2h(p.ctypes.data, ct, p.nbytes), "d2h")
            ctx.check(K.ak_memcpy_d2h(s.ctypes.data, cs, s.nbytes), "d2h")
            self.container = (p, s)
        if own:
            ctx.check(K.ak_synchronize(), "sync")
            ctx.free(ct)
            ctx.free(cs)


def launch(bits, m, k, x, segs, ys, group=128):
    L = AgbLaunch()
    L.bits, L.m, L.nseg, L.k, L.group, L.bf16w = bits, m, len(segs), k, group, 0
    L.x = x.value
    for i, (lin, y) in enumerate(zip(segs, ys)):
        L.wt[i], L.st[i], L.y[i], L.n[i] = lin.wt.value, lin.st.value, y.value, lin.n
    L.use_ldy = 0
    return L


def algo_bytes(L):
    b = 0
    for i in range(L.nseg):
        n = L.n[i]
        b += n * ((L.k + 1023) // 1024 * 1024) * L.bits // 8 + n * ((L.k + 1023) // 1024 * 1024) // L.group * 2
        b += L.m * n * 2
    return b + L.m * L.k * 2


def layer_bits(layer):
    """Per-layer bit width from the seed: W2 p=0.3, W3 p=0.5, W4 p=0.2."""
    u = (np.random.default_rng([SEED, layer]).random())
    return 2 if u < 0.3 else (3 if u < 0.8 else 4)


def build_sweep(ctx, m, cpu_layers, tp=1):
    """64 layers + LM head; returns (plan, meta, containers for the CPU baseline).  tp > 1: one rank's shard of a
    tensor-parallel layer (m1.rs:58-77 tp_rule): q/k/v, gate_up and the LM head by output rows (n / tp), o and down by
    k (k / tp; the all-reduce of their outputs is not part of this one-GPU build).  Each linear reads the output of
    the one before it, as in a decode step: qkv (layer 0: h; later: the previous layer's down) -> o (x = q) -> gate_up
    (x = o) -> down (x = the first k rows of gate_up) -> ..., LM head (x = the last down); the attention, norms and
    residual adds between them are not part of the GEMV path."""
    H, KV, INTER, VOCAB = 5120, 1024, 27648, 152064
    T = tp
    B = ctx.B
    # staging for the containers (largest: LM head 152064 x 5120)
    ct = ctx.alloc(VOCAB * H // 2, keep=False)
    cs = ctx.alloc(VOCAB * H // 128 * 2, keep=False)
    xh = ctx.alloc(m * H * 2)
    ctx.check(B.agb_gen_x(SEED + 1, m * H, 1.0, xh, None), "gen x")
    yq, yk, yv = ctx.alloc(m * H * 2), ctx.alloc(m * KV * 2), ctx.alloc(m * KV * 2)
    yo, yg, ydn = ctx.alloc(m * H * 2), ctx.alloc(m * 2 * INTER * 2), ctx.alloc(m * H * 2)
    ylm = ctx.alloc(m * VOCAB * 2)
    plan, meta, cpu = [], [], []
    xl = xh  # the layer's input
    for l in range(64):
        b = layer_bits(l)
        s = SEED * 1000 + 10 * l
        keep = l < cpu_layers
        q = QLinear(ctx, s + 0, H // T, H, b, ct=ct, cs=cs, keep_container=keep)
        kk = QLinear(ctx, s + 2, KV // T, H, b, ct=ct, cs=cs, keep_container=keep)
        v = QLinear(ctx, s + 4, KV // T, H, b, ct=ct, cs=cs, keep_container=keep)
        o = QLinear(ctx, s + 6, H, H // T, b, ct=ct, cs=cs, keep_container=keep)
        gu = QLinear(ctx, s + 8, 2 * INTER // T, H, b, ct=ct, cs=cs, keep_container=keep)
        dn = QLinear(ctx, s + 10, H, INTER // T, b, ct=ct, cs=cs, keep_container=keep)
        plan += [launch(b, m, H, xl, [q, kk, v], [yq, yk, yv]), launch(b, m, H // T, yq, [o], [yo]),
                 launch(b, m, H, yo, [gu], [yg]), launch(b, m, INTER // T, yg, [dn], [ydn])]
        meta += [("qkv", b), ("o", b), ("gate_up", b), ("down", b)]
        if keep:
            cpu += [(xl, H, [q, kk, v]), (yq, H // T, [o]), (yo, H, [gu]), (yg, INTER // T, [dn])]
        xl = ydn
    lm = QLinear(ctx, SEED * 1000 + 999, VOCAB // T, H, 4, ct=ct, cs=cs)
    plan.append(launch(4, m, H, ydn, [lm], [ylm]))
    meta.append(("lm_head", 4))
    ctx.check(ctx.K.ak_synchronize(), "sync")
    ctx.free(ct)
    ctx.free(cs)
    return plan, meta, cpu


def nlin_layers(cpu, nlin):
    """the number of leading entries of `cpu` that hold the first nlin linears"""
    c = 0
    for i, (_, _, lins) in enumerate(cpu):
        c += len(lins)
        if c >= nlin:
            return i + 1
    return len(cpu)


def cpu_baseline(ctx, m, cpu, budget_s=20.0):
    """The reference's CPU path (reference.rs:53-71, restated in C by the oracle: per-group fp32 sums) on the first
    layers of the same sweep, single thread, timed on this host; GB/s of the same algorithmic bytes."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _lib import oracle, ptr  # the checker / baseline leg (test infrastructure)
    O = oracle()
    K = ctx.K
    xs = {}
    t_total, bytes_total, nlin = 0.0, 0, 0
    for x, k, lins in cpu:
        key = (x.value, k)
        if key not in xs:
            xh = np.zeros(m * k, dtype=np.uint16)
            ctx.check(K.ak_memcpy_d2h(xh.ctypes.data, x, xh.nbytes), "d2h")
            xs[key] = xh
        xh = xs[key]
        for lin in lins:
            p, s = lin.container
            y = np.zeros(m * lin.n, dtype=np.float32)
            t0 = time.perf_counter()
            O.ora_gemv_ref_f32(ptr(xh), m, ptr(p), ptr(s), ptr(y), lin.n, lin.n, k, 128, 1)
            t_total += time.perf_counter() - t0
            bytes_total += lin.wbytes + lin.sbytes + m * lin.n * 2
            nlin += 1
        bytes_total += m * k * 2
        if t_total > budget_s:
            break
    # the same sample on all host cores (rows split statically over threads), reported beside the scalar figure
    nthr = max(1, min(os.cpu_count() or 1, 16))
    t_all = 0.0
    for x, k, lins in cpu[:nlin_layers(cpu, nlin)]:
        xh = xs[(x.value, k)]
        for lin in lins:
            p, s = lin.container
            y = np.zeros(m * lin.n, dtype=np.float32)
            t0 = time.perf_counter()
            O.ora_gemv_ref_f32(ptr(xh), m, ptr(p), ptr(s), ptr(y), lin.n, lin.n, k, 128, nthr)
            t_all += time.perf_counter() - t0
    return {"value": round(bytes_total / t_total / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "all_cores": {"value": round(bytes_total / t_all / 1e9, 3), "cores": nthr},
            "sample": f"{nlin} linears of the sweep's first layers (M={m}), reference CPU path restated in C "
                      f"(oracle/agq_oracle.c ora_gemv_ref_f32, reference.rs:53-71), {t_total:.1f} s"}


def run_sweep(args, K, B):
    ctx = Ctx(K, B)
    cpu_layers = 0 if args.no_cpu else 24  # containers kept on the host for the CPU baseline (about 20 s of it)
    t0 = time.time()
    plan, meta, cpu = build_sweep(ctx, args.m, cpu_layers, args.tp)
    print(f"# sweep generated in {time.time() - t0:.1f} s ({len(plan)} launches)", file=sys.stderr, flush=True)
    arr = (AgbLaunch * len(plan))(*plan)
    total_bytes = sum(algo_bytes(L) for L in plan)
    # one launch per linear (the reference's launch pattern without programmatic launch edges)
    ms_l = ctypes.c_float()
    ctx.check(B.agb_run(arr, len(plan), args.warmup, args.steps, 0 if args.eager else 1, ctypes.byref(ms_l)), "run")
    # the sweep as one chain (ak_wq_chain_run), unless --no-chain
    ms_c, chained, status = ctypes.c_float(), ctypes.c_int(0), ctypes.c_int(0)
    use_chain = not args.no_chain
    if use_chain:
        ctx.check(B.agb_run_chain(arr, len(plan), args.warmup, args.steps, 0 if args.eager else 1, ctypes.byref(ms_c),
                                  ctypes.byref(chained), ctypes.byref(status)), "chain run")
        if status.value != 0:
            raise RuntimeError(f"chained sweep: ak_wq_chain_status() = {status.value} (a bounded wait ran out)")
        use_chain = chained.value == 1
    # the headline is the faster of the two ways to run the same steps in order (both are timed the same way)
    chain_us = round(ms_c.value * 1e3, 1) if use_chain else None
    use_chain = use_chain and ms_c.value < ms_l.value
    ms = ms_c if use_chain else ms_l
    gbs = total_bytes / (ms.value * 1e-3) / 1e9
    # per launch class (linear, bit width; one kernel instance per shape): its launches of the sweep replayed alone
    # as one graph, back to back like in the sweep; the class with the most time is the dominant kernel
    classes = {}
    for L, (name, b) in zip(plan, meta):
        classes.setdefault(f"{name}_w{b}", []).append(L)
    by_kernel = {}
    for key, ls in classes.items():
        sub = (AgbLaunch * len(ls))(*ls)
        t = ctypes.c_float()
        ctx.check(B.agb_run(sub, len(ls), 1, 5, 0 if args.eager else 1, ctypes.byref(t)), "class run")
        by_kernel[key] = {"ms": t.value, "bytes": sum(algo_bytes(L) for L in ls), "launches": len(ls)}
    dom_name, dom = max(by_kernel.items(), key=lambda kv: kv[1]["ms"])
    # the kernel the default routing gives the dominant class (down: k = 27648, the others k = 5120)
    dom_k = 27648 // args.tp if dom_name.startswith("down") else 5120
    dom_kernel = ("i8_m1d_kernel" if args.m <= 2 else "mm_kernel" if args.m >= 17 and dom_k <= 8192
                  else "i8_mt_kernel")
    achieved = dom["bytes"] / (dom["ms"] * 1e-3) / 1e9
    detail = {k: {"launches": v["launches"], "us_each": round(v["ms"] * 1e3 / v["launches"], 2),
                  "GBps": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1)} for k, v in sorted(by_kernel.items())}
    read_bw = ctypes.c_float()
    ctx.check(B.agb_read_bw(4 << 30, 5, ctypes.byref(read_bw)), "read bw")
    cpu_res = cpu_baseline(ctx, args.m, cpu) if cpu else None
    bits_mix = {f"w{b}": sum(1 for (_, bb) in meta[:-1] if bb == b) // 4 for b in (2, 3, 4)}
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic.json")  # HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE
    if args.m == 1 and args.tp == 1 and os.path.exists(tf):
        try:
            traffic = json.load(open(tf)).get(dom_name, {}).get("bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    if use_chain:  # the dominant (only) kernel is the chained launch: one dispatch per sweep
        ctraffic = None
        if args.m == 1 and args.tp == 1 and os.path.exists(tf):
            try:
                ctraffic = json.load(open(tf)).get("chain_sweep", {}).get("bytes_per_launch")
            except (OSError, ValueError):
                ctraffic = None
        ckern = "i8_chain_kernel" if args.m <= 2 else "i8_mt_chain_kernel"
        roof = {"bound": "hbm", "kernel": f"{ckern} (whole sweep, one dispatch)", "achieved": round(gbs, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": ctraffic,
                "launches": 1, "avg_us": round(ms.value * 1e3, 1), "bytes_per_launch": total_bytes}
    else:
        roof = {"bound": "hbm", "kernel": f"{dom_kernel} ({dom_name})", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "launches": dom["launches"], "avg_us": round(dom["ms"] * 1e3 / dom["launches"], 2),
                "bytes_per_launch": dom["bytes"] // dom["launches"]}
    out = {
        "metric": f"effective HBM GB/s (% of peak) + us per 64-layer 32B decode GEMV sweep, M={args.m}",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms.value, 4), "us_per_sweep": round(ms.value * 1e3, 1),
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 MFMA (exact int32 group sums) + fp32 accumulate; bf16 in/out",
        "data": "synthetic (device-generated int4 container, repacked by ak_wq_repack_kt; uniform random codes; "
                "scales |N(0,1)|/sqrt(k E[q^2]) + 1e-6 (not |N(0,1)|*0.02 + 1e-4: keeps the activations unit-sized "
                "through the chained data flow; no effect on timing); each linear reads the previous one's output)",
        "config": {"workload": "64-layer 32B decode GEMV sweep: QKV 5120->7168 (q/k/v segments), O 5120->5120, "
                               "gate_up 5120->55296, down 27648->5120, mixed W2/W3/W4 g128 per layer, "
                               "+ W4 LM head 5120->152064",
                   "m": args.m, "layers_by_bits": bits_mix, "launches": len(plan),
                   "bytes_per_sweep": total_bytes, "graph": not args.eager, "parallelism": "single GPU" if args.tp == 1 else f"one rank of tp{args.tp}: per-rank shapes, no all-reduce",
                   "chained": use_chain},
        "roofline": roof,
        "chained_launch": {"us_per_sweep": chain_us,
                           "GBps": round(total_bytes / (chain_us * 1e-6) / 1e9, 1) if chain_us else None},
        "one_launch_per_linear": {"us_per_sweep": round(ms_l.value * 1e3, 1),
                                  "GBps": round(total_bytes / (ms_l.value * 1e-3) / 1e9, 1),
                                  "dominant_class": {"kernel": f"{dom_kernel} ({dom_name})",
                                                     "GBps": round(achieved, 1), "launches": dom["launches"],
                                                     "avg_us": round(dom["ms"] * 1e3 / dom["launches"], 2),
                                                     "bytes_per_launch": dom["bytes"] // dom["launches"],
                                                     "traffic": traffic}},
        "stream_read_ceiling_GBps": round(read_bw.value, 1),
        "per_linear": detail,
        "cpu_baseline": cpu_res,
    }
    ctx.free_all()
    return out


def run_single(args, K, B):
    """one GEMV shape, weights rotated over >= 1 GB of copies (beats the 256 MB cache)."""
    ctx = Ctx(K, B)
    cfgs = {0: [(4, [5120], 5120, 1.0)], 1: [(3, [55296], 5120, 1.0)], 2: [(2, [5120], 27648, 0.5)],
            3: [(4, [5120, 1024, 1024], 5120, 1.0), (4, [5120], 5120, 1.0)]}
    ms_list = [args.m] if args.config != 3 else [1, 2, 4, 8, 16] if args.m == 1 else [args.m]
    lines = []
    for bits, ns, k, xs in cfgs[args.config]:
        for m in ms_list:
            one = sum(K.ak_wq_kt_weight_bytes(bits, n, k) + K.ak_w4_kt_scale_bytes(n, k, 128) for n in ns)
            copies = max(2, (1 << 30) // one + 1)
            lins = [[QLinear(ctx, SEED + 100 * c + i, n, k, bits) for i, n in enumerate(ns)] for c in range(copies)]
            x = ctx.alloc(m * k * 2)
            ctx.check(B.agb_gen_x(SEED + 7, m * k, xs, x, None), "gen x")
            ys = [ctx.alloc(m * n * 2) for n in ns]
            plan = [launch(bits, m, k, x, lins[c], ys) for c in range(copies)]
            arr = (AgbLaunch * len(plan))(*plan)
            t = ctypes.c_float()
            steps = max(1, (args.steps * 10 + copies - 1) // copies)
            ctx.check(B.agb_run(arr, len(plan), args.warmup, steps, 0 if args.eager else 1, ctypes.byref(t)), "run")
            us = t.value * 1e3 / copies
            by = algo_bytes(plan[0])
            flops = 2.0 * m * sum(ns) * k  # algorithmic multiply-adds x 2
            lines.append({"config": args.config, "bits": bits, "n": ns, "k": k, "m": m, "us": round(us, 2),
                          "GBps": round(by / (us * 1e-6) / 1e9, 1), "pct_of_peak": round(100 * by / (us * 1e-6) / 1e9
                                                                                         / HBM_PEAK_GBS, 2),
                          "TOPS": round(flops / (us * 1e-6) / 1e12, 2),
                          "mfma_util_int8": round(flops / (us * 1e-6) / INT8_PEAK_OPS, 5),
                          "bytes": by, "copies": copies, "graph": not args.eager})
            ctx.free_all()
    return lines


def run_i8(args, K, B):
    """The INT8 LM head GEMV (ak_i8_gemv; reference i8_gemv.cu): 152064 x 5120 int8 weights with fp32 row scales,
    M = 1, 4, 16 tokens; two weight copies in turn (each 778 MB, beyond the 256 MB cache)."""
    ctx = Ctx(K, B)
    n, k, copies = 152064, 5120, 2
    w = ctx.alloc(copies * n * k)
    sc = ctx.alloc(copies * n * 4)
    ctx.check(B.agb_gen_i8(SEED + 31, copies * n * k, w, None), "gen i8")
    ctx.check(B.agb_gen_f32(SEED + 32, copies * n, 0.02 * 3 / 127, 1e-6, sc, None), "gen scales")
    lines = []
    for m in ([args.m] if args.m != 1 else [1, 4, 16]):
        x = ctx.alloc(m * k * 2)
        y = ctx.alloc(m * n * 2)
        ctx.check(B.agb_gen_x(SEED + 33, m * k, 1.0, x, None), "gen x")
        t = ctypes.c_float()
        ctx.check(B.agb_time_i8_gemv(x, w, sc, y, m, n, k, copies, args.warmup, max(args.steps, 10),
                                     ctypes.byref(t)), "i8 gemv")
        us = t.value * 1e3
        by = n * k + n * 4 + m * k * 2 + m * n * 2
        lines.append({"config": "i8_lm_head", "n": n, "k": k, "m": m, "us": round(us, 2),
                      "GBps": round(by / (us * 1e-6) / 1e9, 1),
                      "pct_of_peak": round(100 * by / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2), "bytes": by,
                      "copies": copies, "graph": True})
    ctx.free_all()
    return lines


def run_xover(args, K, B):
    """The GEMV-versus-GEMM crossover in M: the quantized GEMV (ak_wq_gemv_kt_multi, M <= 128) against the prefill
    route (ak_wq_dequant_kt_rows of the whole weight, then the bf16 library GEMM ak_bf16_linear_f32reduce; the
    reference's route above 128 tokens, m1_model.cu:1876-1897) on gate_up W3 (55296 x 5120), o W4 (5120 x 5120) and
    down W2 (5120 x 27648); weights rotated over copies beyond the 256 MB cache.  Eager calls, HIP events."""
    ctx = Ctx(K, B)
    vp = ctypes.c_void_p
    B.agb_time_xover.argtypes = [ctypes.c_int, vp, ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.c_int,
                                 vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.POINTER(ctypes.c_float)]
    B.agb_time_xover.restype = ctypes.c_int
    ms_list = [1, 2, 4, 8, 16, 32, 64, 128, 256, 512]
    K.ak_wq_set_mm_min.restype, K.ak_wq_set_mm_min.argtypes = ctypes.c_int, [ctypes.c_int]
    lines = []
    for name, bits, n, k in (("gate_up_w3", 3, 55296, 5120), ("o_w4", 4, 5120, 5120), ("down_w2", 2, 5120, 27648),
                             ("qkv_w4", 4, 7168, 5120), ("lm_head_w4", 4, 152064, 5120)):
        lins = []
        while sum(L.wbytes for L in lins) < 400e6:
            lins.append(QLinear(ctx, SEED * 1000 + 700 + len(lins), n, k, bits))
        wts = (vp * len(lins))(*[L.wt for L in lins])
        sts = (vp * len(lins))(*[L.st for L in lins])
        mmax = ms_list[-1]
        x = ctx.alloc(mmax * k * 2)
        y = ctx.alloc(mmax * n * 2)
        wd = ctx.alloc(n * k * 2)
        ctx.check(B.agb_gen_x(SEED + 41, mmax * k, 1.0, x, None), "gen x")
        row = {"config": "xover", "linear": name, "bits": bits, "n": n, "k": k, "copies": len(lins),
               "us_gemv": {}, "us_dequant_gemm": {}, "us_fused_gemm": {}}
        for m in ms_list:
            t = ctypes.c_float()
            if m <= 128:
                ctx.check(B.agb_time_xover(bits, x, m, wts, sts, len(lins), wd, y, n, k, 0, 3, 20, ctypes.byref(t)),
                          "gemv")
                row["us_gemv"][m] = round(t.value * 1e3, 2)
                if m >= 2:  # the two GEMV routes of the default numerics (bit-identical), each forced
                    for key, mmin in (("us_gemv_integer", 0), ("us_gemv_mfma", 2)):
                        K.ak_wq_set_mm_min(mmin)
                        ctx.check(B.agb_time_xover(bits, x, m, wts, sts, len(lins), wd, y, n, k, 0, 3, 20,
                                                   ctypes.byref(t)), "gemv route")
                        row.setdefault(key, {})[m] = round(t.value * 1e3, 2)
                    K.ak_wq_set_mm_min(-1)
            ctx.check(B.agb_time_xover(bits, x, m, wts, sts, len(lins), wd, y, n, k, 1, 2, 10, ctypes.byref(t)),
                      "dequant + gemm")
            row["us_dequant_gemm"][m] = round(t.value * 1e3, 2)
            ctx.check(B.agb_time_xover(bits, x, m, wts, sts, len(lins), wd, y, n, k, 2, 2, 10, ctypes.byref(t)),
                      "fused gemm")
            row["us_fused_gemm"][m] = round(t.value * 1e3, 2)
        faster = [m for m in row["us_gemv"] if row["us_dequant_gemm"][m] < row["us_gemv"][m]]
        row["crossover_m"] = min(faster) if faster else None
        lines.append(row)
        ctx.free_all()
    return lines


def run_prefill(args, K, B):
    """The prefill GEMM above 128 tokens: the fused dequantize-in-GEMM kernel (ak_wq_gemm_kt) against the reference's
    route (ak_wq_dequant_kt_rows of the whole weight, then the library GEMM ak_bf16_linear_f32reduce;
    m1_model.cu:1876-1897) on the 32B shapes at 512 and 2048 tokens; weights rotated over >= 400 MB of copies, eager
    calls, HIP events.  TFLOP/s = 2 m n k / time, against the 2.5 PFLOP/s bf16 dense peak."""
    ctx = Ctx(K, B)
    vp = ctypes.c_void_p
    B.agb_time_xover.argtypes = [ctypes.c_int, vp, ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.c_int,
                                 vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.POINTER(ctypes.c_float)]
    B.agb_time_xover.restype = ctypes.c_int
    lines = []
    for name, bits, n, k in (("gate_up_w3", 3, 55296, 5120), ("down_w2", 2, 5120, 27648), ("qkv_w4", 4, 7168, 5120),
                             ("o_w4", 4, 5120, 5120), ("lm_head_w4", 4, 152064, 5120)):
        lins = []
        while sum(L.wbytes for L in lins) < 400e6:
            lins.append(QLinear(ctx, SEED * 1000 + 900 + len(lins), n, k, bits))
        wts = (vp * len(lins))(*[L.wt for L in lins])
        sts = (vp * len(lins))(*[L.st for L in lins])
        ms = (512, 2048)
        x = ctx.alloc(max(ms) * k * 2)
        y = ctx.alloc(max(ms) * n * 2)
        wd = ctx.alloc(n * k * 2)
        ctx.check(B.agb_gen_x(SEED + 43, max(ms) * k, 1.0, x, None), "gen x")
        for m in ms:
            row = {"config": "prefill", "linear": name, "bits": bits, "n": n, "k": k, "m": m, "copies": len(lins)}
            for key, mode in (("fused", 2), ("dequant_gemm", 1)):
                t = ctypes.c_float()
                ctx.check(B.agb_time_xover(bits, x, m, wts, sts, len(lins), wd, y, n, k, mode, 2,
                                           max(5, min(args.steps, 10)), ctypes.byref(t)), key)
                us = t.value * 1e3
                tf = 2.0 * m * n * k / (us * 1e-6) / 1e12
                row[key] = {"us": round(us, 1), "TFLOPs": round(tf, 1), "frac_bf16_peak": round(tf / 2500.0, 3)}
            lines.append(row)
        ctx.free_all()
    return lines


def run_bi(args, K, B):
    """The batch-invariant bf16 GEMV (ak_bf16_gemv_bi; reference bi_gemv.cu): a 5120 x 5120 bf16 weight (weights
    rotated over >= 1 GB of copies) and a small-n projection (48 x 5120), M = 1, 16, 128."""
    ctx = Ctx(K, B)
    lines = []
    for n, k in ((5120, 5120), (48, 5120)):
        one = n * k * 2
        copies = max(2, (1 << 30) // one + 1)
        w = ctx.alloc(copies * one)
        ctx.check(B.agb_gen_x(SEED + 41, copies * n * k, 0.02, w, None), "gen w")
        for m in (1, 16, 128):
            x, y = ctx.alloc(m * k * 2), ctx.alloc(m * n * 2)
            ctx.check(B.agb_gen_x(SEED + 42, m * k, 1.0, x, None), "gen x")
            t = ctypes.c_float()
            ctx.check(B.agb_time_bi_gemv(x, w, y, m, n, k, copies, args.warmup, max(args.steps, 20), ctypes.byref(t)),
                      "bi gemv")
            us = t.value * 1e3
            by = n * k * 2 + m * k * 2 + m * n * 2
            lines.append({"config": "bf16_gemv_bi", "n": n, "k": k, "m": m, "us": round(us, 2),
                          "GBps": round(by / (us * 1e-6) / 1e9, 1),
                          "pct_of_peak": round(100 * by / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                          "TFLOPs": round(2.0 * m * n * k / (us * 1e-6) / 1e12, 2), "copies": copies, "graph": True})
        ctx.free_all()
    return lines


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--tp", type=int, default=1, choices=[1, 2, 4, 8],
                    help="sweep over one rank's shard of a tensor-parallel decode layer (not the headline)")
    ap.add_argument("--config", default="sweep")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true")
    ap.add_argument("--no-chain", action="store_true", help="time the sweep as one launch per linear only")
    ap.add_argument("--exact", action="store_true", help="the reference's exact fp32 numerics instead")
    ap.add_argument("--calib", action="store_true",
                    help="first copy 256 MiB with a plain copy kernel (the known-size reference for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the GEMV would shard by output rows with "
              "no communication, or by k with one all-reduce of the outputs). Run with --gpus 1.", file=sys.stderr)
        return 2
    K, B = load_libs()
    for fn in ("ak_w4_set_lean", "ak_w4_set_mma"):
        getattr(K, fn).argtypes, getattr(K, fn).restype = [ctypes.c_int], ctypes.c_int
    if args.exact:
        K.ak_w4_set_mma(0)
    name = ctypes.create_string_buffer(128)
    K.ak_device_name(0, name, 128)
    print(f"# device {name.value.decode()}", file=sys.stderr, flush=True)
    if args.calib:
        B.agb_copy.argtypes, B.agb_copy.restype = [ctypes.c_size_t, ctypes.c_int], ctypes.c_int
        if B.agb_copy(256 << 20, 2):
            raise RuntimeError("calibration copy failed")
    if args.config == "sweep":
        print(json.dumps(run_sweep(args, K, B)), flush=True)
    elif args.config == "bi":
        for line in run_bi(args, K, B):
            print(json.dumps(line), flush=True)
    elif args.config == "xover":
        for line in run_xover(args, K, B):
            print(json.dumps(line), flush=True)
    elif args.config == "prefill":
        for line in run_prefill(args, K, B):
            print(json.dumps(line), flush=True)
    elif args.config == "i8":
        for line in run_i8(args, K, B):
            print(json.dumps(line), flush=True)
    else:
        args.config = int(args.config)
        for line in run_single(args, K, B):
            print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
