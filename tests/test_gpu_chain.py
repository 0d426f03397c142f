"""Chained GEMV steps (ak_wq_chain_*) on the GPU: one persistent launch that runs a list of ak_wq_gemv_kt_multi steps
(1..2 tokens: the line-load kernel's steps; 3..4 tokens: the tokens-in-A-rows kernel's) with grid barriers or tagged
activations between them (the MI355X counterpart of the reference's programmatic-dependent-launch chains of
GEMV kernels, kernels/src/runtime.cu:198-230, kernels/include/agens_pdl.cuh:1-16).

Every step here reads what the step before it wrote (decoder-layer data flow: qkv -> o -> gate_up -> down -> next
layer), so a missing or leaky barrier, or a stale (non-coherent) read of another XCD's output, changes the results.
Bar: bit-identical to the oracle's default numerics applied step by step, and to one ak_wq_gemv_kt_multi launch per
step.
"""
import ctypes
import os

import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, gemv, gen_container, gen_scales, gen_x, ora_repack, ora_fast, wq_step,
                  Chain)

pytestmark = pytest.mark.gpu

# E[q^2] of uniform codes q in [-2^(b-1), 2^(b-1) - 1]: scales |N(0,1)| * sa with sa = 1 / sqrt(k E[q^2]) keep the
# outputs of a long chain at about unit size
EQ2 = {4: 21.5, 3: 5.5, 2: 1.5}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    K.ak_w4_set_mma(1)
    K.ak_wq_set_mm_min(0)  # the integer-limb kernels at every m (the same numerics as the MFMA route)
    assert K.ak_wq_chain_status() == 0
    yield K
    K.ak_w4_set_mma(-1)
    K.ak_wq_set_mm_min(-1)


class Lin:
    """A linear with its host KT copy (for the oracle)."""

    def __init__(self, seed, n, k, bits, group=128):
        lo, span = -(1 << (bits - 1)), 1 << bits
        packed = gen_container(seed, n, k, lo, span)
        scales = gen_scales(seed + 1, n * k // group, 1.0 / np.sqrt(k * EQ2[bits]), 1e-6)
        self.L = Linear(packed, scales, n, k, group, bits)
        check(self.L.rc, "repack")
        rc, self.wt, self.st = ora_repack(bits, packed, scales, n, k, group)
        assert rc == 0
        self.n, self.k, self.bits, self.group = n, k, bits, group


def layer_plan(seed, bits, H, KV, INTER, group=128):
    q, kk, v = Lin(seed, H, H, bits, group), Lin(seed + 2, KV, H, bits, group), Lin(seed + 4, KV, H, bits, group)
    o, gu, dn = Lin(seed + 6, H, H, bits, group), Lin(seed + 8, 2 * INTER, H, bits, group), \
        Lin(seed + 10, H, INTER, bits, group)
    return [q, kk, v], o, gu, dn


def build(m, layers, H, KV, INTER, group=128):
    """Steps of `layers` decoder layers: qkv(x=h) -> o(x=q) -> gate_up(x=o) -> down(x=gate_up[:INTER]) -> h."""
    h = Dev(m * H * 2)
    steps, flow = [], []  # flow: (step's linears, x buffer, k, outputs)
    x = h
    for li, bits in enumerate(layers):
        qkv, o, gu, dn = layer_plan(1000 + 37 * li, bits, H, KV, INTER, group)
        yq, yk, yv = Dev(m * H * 2), Dev(m * KV * 2), Dev(m * KV * 2)
        yo, ygu, yh = Dev(m * H * 2), Dev(m * 2 * INTER * 2), Dev(m * H * 2)
        for lins, xin, k, ys in [(qkv, x, H, [yq, yk, yv]), ([o], yq, H, [yo]), ([gu], yo, H, [ygu]),
                                 ([dn], ygu, INTER, [yh])]:
            steps.append(wq_step(bits, xin, m, [l.L for l in lins], ys, k, group))
            flow.append((lins, xin, k, ys))
        x = yh
    return h, steps, flow


def oracle_flow(h_host, m, flow):
    """The oracle applied step by step: expected outputs of every step (a dict buffer id -> flat uint16)."""
    vals = {}
    first_x = flow[0][1]
    vals[id(first_x)] = h_host
    out = []
    for lins, xin, k, ys in flow:
        xv = vals[id(xin)][: m * k] if id(xin) in vals else None
        assert xv is not None and xv.size == m * k
        res = []
        for l, y in zip(lins, ys):
            r = ora_fast(l.bits, xv, m, l.wt, l.st, l.n, k, l.group).reshape(-1)
            vals[id(y)] = r
            res.append(r)
        out.append(res)
    return out


def read_outputs(m, flow):
    return [[y.get(np.uint16, m * l.n) for l, y in zip(lins, ys)] for lins, _, _, ys in flow]


def zero_outputs(flow):
    for _, _, _, ys in flow:
        for y in ys:
            z = np.zeros(y.nbytes, np.uint8)
            check(kernels().ak_memcpy_h2d(y.p, z.ctypes.data, y.nbytes), "zero")


def assert_same(got, want, what):
    for si, (g, w) in enumerate(zip(got, want)):
        for j, (a, b) in enumerate(zip(g, w)):
            if not np.array_equal(a, b):
                bad = int(np.sum(a != b))
                raise AssertionError(f"{what}: step {si} segment {j}: {bad} of {a.size} outputs differ")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_chain_data_flow_matches_oracle_and_launches(m):
    K = kernels()
    H, KV, INTER = 2048, 256, 2560  # INTER = 2.5 tiles: the padded last tile in down's k
    h, steps, flow = build(m, [3, 2, 4], H, KV, INTER)
    ch = Chain(steps)
    assert ch.chained
    h_host = gen_x(77 + m, m * H)
    check(K.ak_memcpy_h2d(h.p, h_host.ctypes.data, h_host.nbytes), "h2d")
    want = oracle_flow(h_host, m, flow)
    ch.run()
    check(K.ak_synchronize(), "sync")
    assert K.ak_wq_chain_status() == 0
    assert_same(read_outputs(m, flow), want, "chain vs oracle")
    # the same steps one launch each
    zero_outputs(flow)
    for lins, xin, k, ys in flow:
        gemv(lins[0].bits, xin.p, m, [l.L for l in lins], k, 128, ys=ys)
    check(K.ak_synchronize(), "sync")
    assert_same(read_outputs(m, flow), want, "launches vs oracle")


@pytest.mark.parametrize("m", [1, 4])
def test_chain_replays_with_new_inputs(m):
    """Each replay reads the inputs of its own run: a stale read of an earlier run's values would show."""
    K = kernels()
    H, KV, INTER = 1024, 128, 1536
    h, steps, flow = build(m, [4, 3], H, KV, INTER)
    ch = Chain(steps)
    assert ch.chained
    for rep in range(4):
        h_host = gen_x(500 + rep, m * H)
        check(K.ak_memcpy_h2d(h.p, h_host.ctypes.data, h_host.nbytes), "h2d")
        ch.run()
        if rep == 2:  # a plain launch between chained runs (the flag words persist across launches)
            lins, xin, k, ys = flow[0]
            gemv(lins[0].bits, xin.p, m, [l.L for l in lins], k, 128, ys=ys)
            ch.run()
        check(K.ak_synchronize(), "sync")
        assert K.ak_wq_chain_status() == 0
        assert_same(read_outputs(m, flow), oracle_flow(h_host, m, flow), f"replay {rep}")


def test_chain_independent_steps():
    """A: x -> y1, B (independent): x -> y2, C: y1 -> y3, D (independent of C): y2 -> y4."""
    K = kernels()
    k = 2048
    a, b = Lin(11, 2048, k, 3), Lin(13, 1024, k, 4)
    c, d = Lin(15, 512, 2048, 2), Lin(17, 768, 1024, 3)
    x = Dev(k * 2)
    y1, y2, y3, y4 = Dev(2048 * 2), Dev(1024 * 2), Dev(512 * 2), Dev(768 * 2)
    steps = [wq_step(3, x, 1, [a.L], [y1], k), wq_step(4, x, 1, [b.L], [y2], k, independent=1),
             wq_step(2, y1, 1, [c.L], [y3], 2048), wq_step(3, y2, 1, [d.L], [y4], 1024, independent=1)]
    ch = Chain(steps)
    assert ch.chained
    xh = gen_x(99, k)
    check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
    ch.run()
    check(K.ak_synchronize(), "sync")
    assert K.ak_wq_chain_status() == 0
    r1 = ora_fast(3, xh, 1, a.wt, a.st, a.n, k, 128).reshape(-1)
    r2 = ora_fast(4, xh, 1, b.wt, b.st, b.n, k, 128).reshape(-1)
    r3 = ora_fast(2, r1, 1, c.wt, c.st, c.n, 2048, 128).reshape(-1)
    r4 = ora_fast(3, r2, 1, d.wt, d.st, d.n, 1024, 128).reshape(-1)
    for y, r, n, name in [(y1, r1, 2048, "A"), (y2, r2, 1024, "B"), (y3, r3, 512, "C"), (y4, r4, 768, "D")]:
        assert np.array_equal(y.get(np.uint16, n), r), name


def test_chain_fallback_runs_steps_one_launch_each():
    """A group-64 step (and m > 4) cannot run chained: the chain runs one launch per step, same results."""
    K = kernels()
    H, KV, INTER = 1024, 128, 1024
    for group, m in [(64, 1), (64, 4), (128, 5), (128, 9)]:
        h, steps, flow = build(m, [4, 2], H, KV, INTER, group)
        ch = Chain(steps)
        assert not ch.chained
        h_host = gen_x(31, m * H)
        check(K.ak_memcpy_h2d(h.p, h_host.ctypes.data, h_host.nbytes), "h2d")
        ch.run()
        check(K.ak_synchronize(), "sync")
        assert_same(read_outputs(m, flow), oracle_flow(h_host, m, flow), f"fallback group {group} m {m}")


@pytest.mark.parametrize("m", [1, 2, 4])
def test_chain_at_decode_shapes_matches_launches(m):
    """Two 32B-shaped layers (QKV 5120 -> 5120 + 2 x 1024, O, gate_up 5120 -> 55296, down 27648 -> 5120; the down
    steps split k across workgroups): every chained step equals the oracle on its first, middle and last 64 rows of
    every segment, fed with the activations that step read; the chained launch equals one launch per step bit for
    bit, on two runs in a row (the split's counters return to zero)."""
    K = kernels()
    H, KV, INTER = 5120, 1024, 27648
    h, steps, flow = build(m, [3, 2], H, KV, INTER)
    ch = Chain(steps)
    assert ch.chained
    h_host = gen_x(4242, m * H)
    check(K.ak_memcpy_h2d(h.p, h_host.ctypes.data, h_host.nbytes), "h2d")
    ch.run()
    check(K.ak_synchronize(), "sync")
    assert K.ak_wq_chain_status() == 0
    got = read_outputs(m, flow)
    for si, (lins, xin, k, ys) in enumerate(flow):
        xv = h_host if si == 0 else xin.get(np.uint16, m * k)
        for j, l in enumerate(lins):
            y = got[si][j].reshape(m, l.n)
            for r0 in sorted({0, l.n // 2 - 32, l.n - 64}):
                want = ora_fast(l.bits, xv, m, l.wt, l.st, l.n, k, l.group, rows=(r0, r0 + 64))[:, r0:r0 + 64]
                assert np.array_equal(y[:, r0:r0 + 64], want), f"step {si} segment {j} rows {r0}..{r0 + 64}"
    zero_outputs(flow)
    ch.run()
    check(K.ak_synchronize(), "sync")
    assert_same(read_outputs(m, flow), got, "second chained run")
    zero_outputs(flow)
    for lins, xin, k, ys in flow:
        gemv(lins[0].bits, xin.p, m, [l.L for l in lins], k, 128, ys=ys)
    check(K.ak_synchronize(), "sync")
    assert_same(got, read_outputs(m, flow), "chain vs launches")
    # outputs stay finite and non-trivial through the chain (the data flow carries information)
    last = got[-1][0].astype(np.uint32) << 16
    f = last.view(np.float32)
    assert np.all(np.isfinite(f)) and np.std(f) > 0.05


def test_chain_independent_step_after_a_step_most_workgroups_skip():
    """A: x -> y1 (large), B (dependent): y1[:5120] -> y2 with 16 rows (most workgroups have no rows in it), C (independent of
    B): y1 -> y3 on every workgroup.  C reads A's output, so every workgroup must have passed B's wait, also those
    with no rows in B; the same steps one launch each give the reference values.  Two runs in a row."""
    K = kernels()
    k = 5120
    # B: k = 5120 (the first 5120 outputs of A), 16 rows = 4 blocks: 4 workgroups have rows, 252 skip it
    a, b, c = Lin(21, 27648, k, 3), Lin(23, 16, k, 4), Lin(25, 4096, 27648, 2)
    x = Dev(k * 2)
    y1, y2, y3 = Dev(27648 * 2), Dev(16 * 2), Dev(4096 * 2)
    steps = [wq_step(3, x, 1, [a.L], [y1], k), wq_step(4, y1, 1, [b.L], [y2], k),
             wq_step(2, y1, 1, [c.L], [y3], 27648, independent=1)]
    ch = Chain(steps)
    assert ch.chained
    for rep in range(2):
        xh = gen_x(123 + rep, k)
        check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
        ch.run()
        check(K.ak_synchronize(), "sync")
        assert K.ak_wq_chain_status() == 0
        got = [y.get(np.uint16, n) for y, n in ((y1, 27648), (y2, 16), (y3, 4096))]
        for lin, xin, kk, y in ((a, x, k, y1), (b, y1, k, y2), (c, y1, 27648, y3)):
            gemv(lin.bits, xin.p, 1, [lin.L], kk, 128, ys=[y])
        check(K.ak_synchronize(), "sync")
        for g, (y, n, name) in zip(got, ((y1, 27648, "A"), (y2, 16, "B"), (y3, 4096, "C"))):
            assert np.array_equal(g, y.get(np.uint16, n)), f"run {rep} step {name}"


def build_rank(m, layers, tp, H=5120, KV=1024, INTER=27648):
    """Steps of one tensor-parallel rank's decoder layers: qkv (rows / tp, x = h) -> o (k = H / tp, x = the rank's q
    rows) -> gate_up (rows / tp, x = o) -> down (k = INTER / tp, x = the first INTER / tp gate_up rows) -> h."""
    h = Dev(m * H * 2)
    steps, flow = [], []
    x = h
    for li, bits in enumerate(layers):
        s = 3000 + 37 * li
        q, kk, v = Lin(s, H // tp, H, bits), Lin(s + 2, KV // tp, H, bits), Lin(s + 4, KV // tp, H, bits)
        o, gu, dn = Lin(s + 6, H, H // tp, bits), Lin(s + 8, 2 * INTER // tp, H, bits), Lin(s + 10, H, INTER // tp, bits)
        yq, yk, yv = Dev(m * H // tp * 2), Dev(m * KV // tp * 2), Dev(m * KV // tp * 2)
        yo, ygu, yh = Dev(m * H * 2), Dev(m * 2 * INTER // tp * 2), Dev(m * H * 2)
        for lins, xin, k, ys in [([q, kk, v], x, H, [yq, yk, yv]), ([o], yq, H // tp, [yo]), ([gu], yo, H, [ygu]),
                                 ([dn], ygu, INTER // tp, [yh])]:
            steps.append(wq_step(bits, xin, m, [l.L for l in lins], ys, k))
            flow.append((lins, xin, k, ys))
        x = yh
    return h, steps, flow


@pytest.mark.parametrize("m", [1, 2])
def test_chain_at_tp8_rank_shapes_matches_oracle(m):
    """One TP = 8 rank's layers in one chained launch (o at k = 640: one padded tile; down at k = 3456: the last of
    four tiles padded; the down steps split k across workgroups): every step's outputs equal the oracle applied step
    by step, and equal one launch per step."""
    K = kernels()
    h, steps, flow = build_rank(m, [3, 2, 4], 8)
    ch = Chain(steps)
    assert ch.chained
    h_host = gen_x(5150 + m, m * 5120)
    check(K.ak_memcpy_h2d(h.p, h_host.ctypes.data, h_host.nbytes), "h2d")
    want = oracle_flow(h_host, m, flow)
    ch.run()
    check(K.ak_synchronize(), "sync")
    assert K.ak_wq_chain_status() == 0
    assert_same(read_outputs(m, flow), want, "chain vs oracle")
    zero_outputs(flow)
    for lins, xin, k, ys in flow:
        gemv(lins[0].bits, xin.p, m, [l.L for l in lins], k, 128, ys=ys)
    check(K.ak_synchronize(), "sync")
    assert_same(read_outputs(m, flow), want, "launches vs oracle")


def _run_mixed_chain(m, reps, tags):
    """A: x -> y1; B: y1 -> y2 and C: y2 -> y3 (each reads the step just before it: tagged activations); D: y1 -> y4
    (reads A's output, three steps back: a grid-barrier wait, so C signals the flags); E: SiLU(gate) * up of y4 -> y5
    (reads D's output, fused activation: tagged, k split across workgroups; above two tokens E reads y4 as it is, the
    chained kernel of 3..8 tokens taking no fused activation).  Returns every run's outputs."""
    act = 1 if m <= 2 else 0
    K = kernels()
    k, inter = 2048, 16384
    a, b, c = Lin(41, 4096, k, 3), Lin(43, 2048, 4096, 2), Lin(45, 3072, 2048, 4)
    d, e = Lin(47, 2 * inter, 4096, 3), Lin(49, 1024, inter if act else 2 * inter, 2)
    x = Dev(m * k * 2)
    ys = [Dev(m * n * 2) for n in (4096, 2048, 3072, 2 * inter, 1024)]
    steps = [wq_step(3, x, m, [a.L], [ys[0]], k), wq_step(2, ys[0], m, [b.L], [ys[1]], 4096),
             wq_step(4, ys[1], m, [c.L], [ys[2]], 2048), wq_step(3, ys[0], m, [d.L], [ys[3]], 4096),
             wq_step(2, ys[3], m, [e.L], [ys[4]], inter if act else 2 * inter, act=act)]
    old = os.environ.get("AK_CHAIN_TAGS")
    os.environ["AK_CHAIN_TAGS"] = "1" if tags else "0"
    try:
        ch = Chain(steps)
    finally:
        if old is None:
            del os.environ["AK_CHAIN_TAGS"]
        else:
            os.environ["AK_CHAIN_TAGS"] = old
    assert ch.chained
    runs = []
    for rep in range(reps):
        xh = gen_x(700 + rep, m * k)
        check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
        for y in ys:  # outputs the chain does not write would show
            z = np.zeros(y.nbytes, np.uint8)
            check(K.ak_memcpy_h2d(y.p, z.ctypes.data, y.nbytes), "zero")
        ch.run()
        check(K.ak_synchronize(), "sync")
        assert K.ak_wq_chain_status() == 0
        got = [y.get(np.uint16, m * n) for y, n in zip(ys, (4096, 2048, 3072, 2 * inter, 1024))]
        # the same steps one launch each
        for lin, xin, kk, y in ((a, x, k, ys[0]), (b, ys[0], 4096, ys[1]), (c, ys[1], 2048, ys[2]),
                                (d, ys[0], 4096, ys[3])):
            gemv(lin.bits, xin.p, m, [lin.L], kk, 128, ys=[y])
        if act:
            check(K.ak_wq_gemv_kt_silu(2, ys[3].p, m, e.L.wt.p, e.L.st.p, ys[4].p, 1024, 0, inter, 128, None), "silu")
        else:
            gemv(e.bits, ys[3].p, m, [e.L], 2 * inter, 128, ys=[ys[4]])
        check(K.ak_synchronize(), "sync")
        for si, (g, y, n) in enumerate(zip(got, ys, (4096, 2048, 3072, 2 * inter, 1024))):
            assert np.array_equal(g, y.get(np.uint16, m * n)), f"m={m} run {rep} step {'ABCDE'[si]}"
        runs.append(got)
    return runs


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_chain_tagged_and_barrier_waits_mix(m):
    """Tagged activation waits beside grid-barrier waits in one chain, on three runs in a row with new inputs (the
    launch tag advances; a stale tag of the run before would read old activations): every step equals one launch per
    step, and the chain without tagged waits (AK_CHAIN_TAGS=0) gives the same bits."""
    tagged = _run_mixed_chain(m, 3, True)
    plain = _run_mixed_chain(m, 1, False)
    for si, (g, w) in enumerate(zip(tagged[0], plain[0])):
        assert np.array_equal(g, w), f"step {'ABCDE'[si]}: tagged and barrier-only chains differ"


def test_chain_tagged_read_of_a_later_segment():
    """A: x -> (y0, y1, y2) in three segments; B reads y1 (segment 1: the tagged copy of a later segment); C reads
    B's output with 2 tokens' rows as the step before it produced them.  Chained (with and without tagged
    activations) equals one launch per step, on two runs in a row."""
    K = kernels()
    k, m = 2048, 2
    a = [Lin(81 + i, n, k, 3) for i, n in enumerate((1024, 3072, 512))]
    b, c = Lin(85, 2048, 3072, 4), Lin(87, 640, 2048, 2)
    x = Dev(m * k * 2)
    ya = [Dev(m * L.n * 2) for L in a]
    yb, yc = Dev(m * 2048 * 2), Dev(m * 640 * 2)
    steps = [wq_step(3, x, m, [L.L for L in a], ya, k), wq_step(4, ya[1], m, [b.L], [yb], 3072),
             wq_step(2, yb, m, [c.L], [yc], 2048)]
    for tags in ("1", "0"):
        old = os.environ.get("AK_CHAIN_TAGS")
        os.environ["AK_CHAIN_TAGS"] = tags
        try:
            ch = Chain(steps)
        finally:
            if old is None:
                del os.environ["AK_CHAIN_TAGS"]
            else:
                os.environ["AK_CHAIN_TAGS"] = old
        assert ch.chained
        for rep in range(2):
            xh = gen_x(900 + rep, m * k)
            check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
            ch.run()
            check(K.ak_synchronize(), "sync")
            assert K.ak_wq_chain_status() == 0
            got = [y.get(np.uint16, m * n) for y, n in ((yb, 2048), (yc, 640))]
            gemv(3, x.p, m, [L.L for L in a], k, 128, ys=ya)
            gemv(4, ya[1].p, m, [b.L], 3072, 128, ys=[yb])
            gemv(2, yb.p, m, [c.L], 2048, 128, ys=[yc])
            check(K.ak_synchronize(), "sync")
            for g, (y, n, name) in zip(got, ((yb, 2048, "B"), (yc, 640, "C"))):
                assert np.array_equal(g, y.get(np.uint16, m * n)), f"tags {tags} run {rep} step {name}"


@pytest.mark.parametrize("m", [1, 4])
def test_chain_tag_wraps_after_65536_runs(m):
    """The 16-bit launch tag of tagged activations wraps after 65536 launches of a chain: the runs around the wrap
    (tag 65535, 0, 1) read their own activations, not the previous run's (each run gets new inputs; equal to one
    launch per step)."""
    K = kernels()
    k = 1024
    a, b = Lin(91, 1024, k, 3), Lin(93, 512, 1024, 4)
    x = Dev(m * k * 2)
    y1, y2 = Dev(m * 1024 * 2), Dev(m * 512 * 2)
    ch = Chain([wq_step(3, x, m, [a.L], [y1], k), wq_step(4, y1, m, [b.L], [y2], 1024)])
    assert ch.chained
    xh = gen_x(950, m * k)
    check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
    for _ in range(65534):  # runs 0 .. 65533 (tags 1 .. 65534)
        ch.run()
    check(K.ak_synchronize(), "sync")
    assert K.ak_wq_chain_status() == 0
    for rep in range(4):  # runs 65534 .. 65537: tags 65535, 0, 1, 2
        xh = gen_x(951 + rep, m * k)
        check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
        ch.run()
        check(K.ak_synchronize(), "sync")
        assert K.ak_wq_chain_status() == 0
        got = [y1.get(np.uint16, m * 1024), y2.get(np.uint16, m * 512)]
        gemv(3, x.p, m, [a.L], k, 128, ys=[y1])
        gemv(4, y1.p, m, [b.L], 1024, 128, ys=[y2])
        check(K.ak_synchronize(), "sync")
        assert np.array_equal(got[0], y1.get(np.uint16, m * 1024)), f"run {65534 + rep}: step 0"
        assert np.array_equal(got[1], y2.get(np.uint16, m * 512)), f"run {65534 + rep}: step 1"


@pytest.mark.parametrize("m", [1, 4])
def test_chain_in_a_graph_replays_with_new_inputs(m):
    """The chained launch captured in a hipGraph (ak_wq_chain_run is capturable and allocates nothing): three replays,
    each after new inputs were copied in with an eager synchronous copy, each equal to one launch per step (the launch
    tag advances inside the kernel, so every replay reads its own tagged activations)."""
    K = kernels()
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    k = 2048
    a, b, c = Lin(101, 2048, k, 3), Lin(103, 1024, 2048, 2), Lin(105, 768, 1024, 4)
    x = Dev(m * k * 2)
    y1, y2, y3 = Dev(m * 2048 * 2), Dev(m * 1024 * 2), Dev(m * 768 * 2)
    ch = Chain([wq_step(3, x, m, [a.L], [y1], k), wq_step(2, y1, m, [b.L], [y2], 2048),
                wq_step(4, y2, m, [c.L], [y3], 1024)])
    assert ch.chained
    stream, graph, exe = vp(), vp(), vp()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        assert hip.hipStreamBeginCapture(stream, ctypes.c_int(1)) == 0  # thread-local capture mode
        rc = K.ak_wq_chain_run(ch.h, stream)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        check(rc, "ak_wq_chain_run under capture")
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        for rep in range(3):
            xh = gen_x(1100 + rep, m * k)
            check(K.ak_memcpy_h2d(x.p, xh.ctypes.data, xh.nbytes), "h2d")
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            assert K.ak_wq_chain_status() == 0
            got = [y.get(np.uint16, m * n) for y, n in ((y1, 2048), (y2, 1024), (y3, 768))]
            gemv(3, x.p, m, [a.L], k, 128, ys=[y1])
            gemv(2, y1.p, m, [b.L], 2048, 128, ys=[y2])
            gemv(4, y2.p, m, [c.L], 1024, 128, ys=[y3])
            check(K.ak_synchronize(), "sync")
            for g, (y, n, name) in zip(got, ((y1, 2048, "A"), (y2, 1024, "B"), (y3, 768, "C"))):
                assert np.array_equal(g, y.get(np.uint16, m * n)), f"replay {rep} step {name}"
    finally:
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(stream)


def test_chained_launches_on_two_streams_are_refused_while_one_runs():
    """Chained launches on one device share its flag words: ak_wq_chain_run refuses (hipErrorNotReady, 600) a launch on
    another stream while the device's last chained launch is still running, and accepts launches on the same stream
    (stream-ordered) and, once the other finished, on the other stream."""
    K = kernels()
    hip = ctypes.CDLL("libamdhip64.so")
    sa, sb = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(sa)) == 0 and hip.hipStreamCreate(ctypes.byref(sb)) == 0
    try:
        k, n = 5120, 55296
        big = Lin(61, n, k, 3)
        x, y = Dev(k * 2), Dev(n * 2)
        # 200 independent steps over one 106 MB weight: a few milliseconds of device time per run
        steps = [wq_step(3, x, 1, [big.L], [y], k, independent=1) for _ in range(200)]
        ch = Chain(steps)
        assert ch.chained
        assert K.ak_wq_chain_run(ch.h, sa) == 0
        assert K.ak_wq_chain_run(ch.h, sb) == 600, "a chained launch on another stream while one runs"
        assert K.ak_wq_chain_run(ch.h, sa) == 0, "the same stream is ordered: accepted"
        assert hip.hipStreamSynchronize(sa) == 0
        assert K.ak_wq_chain_run(ch.h, sb) == 0, "the other stream once the first launch finished"
        assert hip.hipStreamSynchronize(sb) == 0
        assert K.ak_wq_chain_status() == 0
    finally:
        hip.hipStreamDestroy(sa)
        hip.hipStreamDestroy(sb)
