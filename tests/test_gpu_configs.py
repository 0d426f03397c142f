"""BASELINE configs 3 and 4 at their own shapes on the GPU, through the C ABI, against the oracle.

Routing depends on the shape (rows per CU decide split-K, the activation image size decides chunking), so these
run exactly the shapes the benchmark times:
  - config 3: the attention QKV projection as one launch of q / k / v segments (5120 / 1024 / 1024 rows, k = 5120)
    and the O projection (5120 x 5120), W4 g128, M = 2, 4, 8, 16;
  - config 4: two 32B-shaped decoder layers (QKV, O, gate_up 5120 -> 55296, down 27648 -> 5120 with the SiLU(gate) *
    up activation) at M = 4 and 16, each step fed by the one before, and the W4 LM head (152064 x 5120) at M = 1, 4,
    16.
Bar: bit-exact to the oracle's default numerics (ora_gemv_fast_kt) on sampled 64-row windows of every segment
(first, middle, last), within BASELINE's 2e-3 of the reference's fp32 path (reference.rs:53-71) beyond the bf16 output
rounding on 256 rows, and the reference gate's bound vs fp64 (test_w4.cu:123-141).  Reference harness for these
shapes: kernels/bench/test_w4.cu:297-371, kernels/m1/m1_model.cu:2794-2812.
"""
import ctypes

import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, gemv, gen_container, gen_scales, gen_x, ora_repack, ora_fast,
                  ora_ref_f32, ora_ref_f64, max_rel_excess, max_ulp_bound, wq_step, Chain, bf2f_array)

pytestmark = pytest.mark.gpu

H, KV, INTER, VOCAB = 5120, 1024, 27648, 152064


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    K.ak_w4_set_mma(1)
    K.ak_wq_set_mm_min(0)  # the integer-limb kernels at every m (the same numerics as the MFMA route)
    yield K
    K.ak_w4_set_mma(-1)
    K.ak_wq_set_mm_min(-1)


class Lin:
    """A linear on the device and the host container it was repacked from."""

    def __init__(self, seed, n, k, bits, sa=0.02, tile_rows=None):
        lo, span = -(1 << (bits - 1)), 1 << bits
        if tile_rows:  # rows repeat every tile_rows rows (the LM head: 152064 rows at host-generation cost of fewer)
            base = gen_container(seed, tile_rows, k, lo, span).reshape(tile_rows, k // 8)
            reps = (n + tile_rows - 1) // tile_rows
            packed = np.ascontiguousarray(np.tile(base, (reps, 1))[:n]).reshape(-1)
            sb = gen_scales(seed + 1, tile_rows * k // 128, sa, 1e-4).reshape(tile_rows, k // 128)
            scales = np.ascontiguousarray(np.tile(sb, (reps, 1))[:n]).reshape(-1)
        else:
            packed = gen_container(seed, n, k, lo, span)
            scales = gen_scales(seed + 1, n * k // 128, sa, 1e-4)
        self.L = Linear(packed, scales, n, k, 128, bits)
        check(self.L.rc, "repack")
        self.packed, self.scales, self.n, self.k, self.bits = packed, scales, n, k, bits

    def rows(self, r0, r1):
        """KT of rows [r0, r1) (repacked by the oracle from the container: rows are independent)."""
        words = self.k // 8
        p = np.ascontiguousarray(self.packed[r0 * words:r1 * words])
        s = np.ascontiguousarray(self.scales[r0 * (self.k // 128):r1 * (self.k // 128)])
        rc, wt, st = ora_repack(self.bits, p, s, r1 - r0, self.k, 128)
        assert rc == 0
        return p, s, wt, st


def windows(n, w=64):
    return sorted({0, max(0, n // 2 - w // 2), max(0, n - w)})


def check_rows(lin, x, m, y, what, tol_rows=0):
    """y [m][n] (the GPU's outputs) against the oracle on 64-row windows; tolerance checks on tol_rows rows."""
    for r0 in windows(lin.n):
        r1 = min(lin.n, r0 + 64)
        _, _, wt, st = lin.rows(r0, r1)
        want = ora_fast(lin.bits, x, m, wt, st, r1 - r0, lin.k, 128)
        got = y[:, r0:r1]
        if not np.array_equal(got, want):
            bad = np.argwhere(got != want)[:4]
            raise AssertionError(f"{what}: rows {r0}..{r1}: {int(np.sum(got != want))} outputs differ, e.g. {bad}")
    if tol_rows:
        r0 = lin.n // 3
        r1 = r0 + tol_rows
        p, s, _, _ = lin.rows(r0, r1)
        ref32 = ora_ref_f32(x, m, p, s, r1 - r0, lin.k, 128)
        ref64, mag = ora_ref_f64(x, m, p, s, r1 - r0, lin.k, 128)
        assert max_rel_excess(y[:, r0:r1], ref32) <= 2e-3, what
        assert max_ulp_bound(y[:, r0:r1], ref64, mag) <= 1.0, what


@pytest.fixture(scope="module")
def attn():
    q, k, v = Lin(3100, H, H, 4), Lin(3102, KV, H, 4), Lin(3104, KV, H, 4)
    o = Lin(3106, H, H, 4)
    return [q, k, v], o


@pytest.mark.parametrize("m", [2, 4, 8, 16])
def test_config3_qkv_and_o_at_bench_shapes(attn, m):
    qkv, o = attn
    x = gen_x(3200 + m, m * H)
    X = Dev.of(x)
    ys = gemv(4, X, m, [l.L for l in qkv], H, 128)
    for l, Y in zip(qkv, ys):
        y = Y.get(np.uint16, m * l.n).reshape(m, l.n)
        check_rows(l, x, m, y, f"qkv segment n={l.n} m={m}", tol_rows=256 if l.n == H else 0)
        # one segment launched alone gives the same rows (the multi-segment route is not a different numerics)
        (Y1,) = gemv(4, X, m, [l.L], H, 128)
        assert np.array_equal(Y1.get(np.uint16, m * l.n).reshape(m, l.n), y)
    (Yo,) = gemv(4, X, m, [o.L], H, 128)
    check_rows(o, x, m, Yo.get(np.uint16, m * H).reshape(m, H), f"o m={m}", tol_rows=256)


def layer_bits(layer, seed=20261201):
    """The benchmark's per-layer bit widths (W2 p=0.3, W3 p=0.5, W4 p=0.2)."""
    u = np.random.default_rng([seed, layer]).random()
    return 2 if u < 0.3 else (3 if u < 0.8 else 4)


@pytest.mark.parametrize("m,bits,default_route", [(4, None, False), (16, None, False), (16, (2, 3, 4), True),
                                                  (24, (2, 3, 4), True)])
def test_config4_layers_step_by_step(m, bits, default_route):
    """QKV(x = h) -> O(x = q) -> gate_up(x = o) -> down(x = SiLU(gate) * up of gate_up) -> next layer's h, as one
    chain (ak_wq_chain_run) and as one launch per step; every step's outputs equal the oracle applied to the inputs
    that step actually read.  Two layers of the benchmark's bit widths on the integer-limb kernels, and three layers
    (W2, W3, W4) on the library's default routing: at 24 tokens QKV, O and gate_up take the fp16-MFMA kernel and down
    (k = 27648) the integer kernels."""
    K = kernels()
    if default_route:
        K.ak_wq_set_mm_min(-1)
    try:
        run_layers(K, m, bits or [layer_bits(li) for li in range(2)])
    finally:
        K.ak_wq_set_mm_min(0)


def run_layers(K, m, layer_bit_widths):
    steps, flow = [], []
    h = Dev(m * H * 2)
    x = h
    for li, b in enumerate(layer_bit_widths):
        s = 4000 + 50 * li
        eq2 = {4: 21.5, 3: 5.5, 2: 1.5}[b]  # scales ~ 1 / sqrt(k E[q^2]): activations stay about unit size
        qkv = [Lin(s, H, H, b, 1 / np.sqrt(H * eq2)), Lin(s + 2, KV, H, b, 1 / np.sqrt(H * eq2)),
               Lin(s + 4, KV, H, b, 1 / np.sqrt(H * eq2))]
        o = Lin(s + 6, H, H, b, 1 / np.sqrt(H * eq2))
        gu = Lin(s + 8, 2 * INTER, H, b, 1 / np.sqrt(H * eq2))
        dn = Lin(s + 10, H, INTER, b, 1 / np.sqrt(INTER * eq2))
        yq, yk, yv = Dev(m * H * 2), Dev(m * KV * 2), Dev(m * KV * 2)
        yo, ygu, yh = Dev(m * H * 2), Dev(m * 2 * INTER * 2), Dev(m * H * 2)
        for lins, xin, k, ys, act in [(qkv, x, H, [yq, yk, yv], 0), ([o], yq, H, [yo], 0), ([gu], yo, H, [ygu], 0),
                                      ([dn], ygu, INTER, [yh], 1)]:
            steps.append(wq_step(b, xin, m, [l.L for l in lins], ys, k, act=act))
            flow.append((lins, xin, k, ys, act))
        x = yh
    hh = gen_x(4500 + m, m * H)
    check(K.ak_memcpy_h2d(h.p, hh.ctypes.data, hh.nbytes), "h2d")
    ch = Chain(steps)
    ch.run()
    check(K.ak_synchronize(), "sync")
    assert K.ak_wq_chain_status() == 0
    got = [[y.get(np.uint16, m * l.n) for l, y in zip(lins, ys)] for lins, _, _, ys, _ in flow]
    for si, (lins, xin, k, ys, act) in enumerate(flow):
        if act:  # the activation the fused step applies: ak_silu_mul of gate_up, the same value bit for bit
            A = Dev(m * k * 2)
            check(K.ak_silu_mul(xin.p, A.p, m, k, None), "silu_mul")
            xv = A.get(np.uint16, m * k)
        else:
            xv = xin.get(np.uint16, m * k)
        for l, y in zip(lins, got[si]):
            check_rows(l, xv, m, y.reshape(m, l.n), f"step {si} n={l.n} bits={l.bits} m={m}")
    # outputs stay finite and non-trivial through the first two layers (the third layer's SiLU * up products may grow
    # beyond bf16's range; the oracle checks above cover whatever values arise)
    f = bf2f_array(got[7][0])
    assert np.all(np.isfinite(f)) and np.std(f) > 0.05, (np.sum(~np.isfinite(f)), np.std(f[np.isfinite(f)]))
    # one launch per step: the same bits
    for lins, xin, k, ys, act in flow:
        for y in ys:
            check(K.ak_memcpy_h2d(y.p, np.zeros(y.nbytes, np.uint8).ctypes.data, y.nbytes), "zero")
    for lins, xin, k, ys, act in flow:
        if act:
            check(K.ak_wq_gemv_kt_silu(lins[0].bits, xin.p, m, lins[0].L.wt.p, lins[0].L.st.p, ys[0].p, lins[0].n,
                                       0, k, 128, None), "silu gemv")
        else:
            gemv(lins[0].bits, xin.p, m, [l.L for l in lins], k, 128, ys=ys)
    check(K.ak_synchronize(), "sync")
    for si, (lins, _, _, ys, _) in enumerate(flow):
        for j, (l, y) in enumerate(zip(lins, ys)):
            assert np.array_equal(y.get(np.uint16, m * l.n), got[si][j]), f"launches vs chain: step {si} seg {j}"


@pytest.fixture(scope="module")
def lm_head():
    return Lin(4700, VOCAB, H, 4, tile_rows=8192 + 13)


@pytest.mark.parametrize("m", [1, 4, 16])
def test_config4_w4_lm_head(lm_head, m):
    """The W4 LM head (152064 x 5120) through ak_wq_gemv_kt_multi: its route at every M (at 16 tokens a split-K
    launch of about 40 row blocks per CU), rows equal to the oracle including the last rows."""
    x = gen_x(4800 + m, m * H)
    X = Dev.of(x)
    (Y,) = gemv(4, X, m, [lm_head.L], H, 128)
    y = Y.get(np.uint16, m * VOCAB).reshape(m, VOCAB)
    check_rows(lm_head, x, m, y, f"lm head m={m}", tol_rows=256)
    # rows repeat with the container's period: a wrong row or tile index in a far block would break the repeat
    p = 8192 + 13
    assert np.array_equal(y[:, VOCAB - 64:], y[:, VOCAB - 64 - 18 * p:VOCAB - 18 * p])
