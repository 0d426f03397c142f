"""Every launch configuration of the one- and two-token GEMV gives the same bits: each stripe-set split (1, 2, 4, 8)
with 16 or 8 waves per workgroup, forced through ak_wq_tune_override, against the oracle (ora_gemv_fast_kt) bit for
bit, on shapes with padded rows and tiles, several segments, long k and both token counts.  The reference's tuner makes
the same check of its variants (kernels/bench/tune_w4.cu:1-91)."""
import ctypes

import numpy as np
import pytest

from _lib import kernels, check, Dev, Linear, gemv, gen_container, gen_scales, gen_x, ora_fast

pytestmark = pytest.mark.gpu

SHAPES = [  # bits, segment rows, k
    (3, [5120, 1024, 1024], 5120),
    (2, [1001], 3072),
    (4, [300, 77], 2176),
    (3, [640], 27648),
    (2, [5120], 8192),
]
CONFIGS = [(sp, nw) for nw in (16, 8) for sp in (1, 2, 4, 8)]


@pytest.fixture(scope="module")
def K():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    K.ak_wq_tune_override.argtypes = [ctypes.c_int] * 3
    K.ak_wq_set_mm_min(0)  # the integer-limb kernels at every m (the same numerics as the MFMA route)
    yield K
    K.ak_wq_tune_override(0, 0, -1)
    K.ak_wq_set_mm_min(-1)


@pytest.mark.parametrize("bits,ns,k", SHAPES)
@pytest.mark.parametrize("m", [1, 2])
def test_every_split_is_bit_exact(K, bits, ns, k, m):
    lo, span = -(1 << (bits - 1)), 1 << bits
    lins = []
    for j, n in enumerate(ns):
        L = Linear(gen_container(3100 + 7 * j + bits, n, k, lo, span), gen_scales(3200 + j, n * k // 128), n, k, 128,
                   bits)
        check(L.rc)
        lins.append(L)
    x = gen_x(3300 + m, m * k)
    X = Dev.of(x)
    want = []
    for L in lins:
        wt, st = L.host_kt()
        want.append(ora_fast(bits, x, m, wt, st, L.n, k, 128))
    try:
        for sp, nw in CONFIGS:
            K.ak_wq_tune_override(sp, nw, 0)
            ys = gemv(bits, X, m, lins, k, 128)
            for L, Y, w in zip(lins, ys, want):
                got = Y.get(np.uint16, m * L.n).reshape(m, L.n)
                bad = int(np.sum(got != w))
                assert bad == 0, f"split {sp} nwv {nw}: {bad} of {m * L.n} outputs differ (W{bits} n={L.n} k={k})"
    finally:
        K.ak_wq_tune_override(0, 0, -1)
