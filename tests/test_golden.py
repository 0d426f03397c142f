"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the reference tests' generators,
kernels/bench/test_w4.cu:36-40, 75-77 and kernels/bench/test_wq.cu:36-40, 75-90).

CPU: the generator restatement reproduces the stored inputs, the oracle reproduces the stored outputs, and the stored
GEMV outputs meet the reference's bound against fp64 (test_w4.cu:123-141) and the 2e-3 tolerance.
GPU: the HIP repack, dequantization and both GEMV numerics reproduce the stored bytes through the C ABI.
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import _lib as L  # noqa: E402
import make_golden as G  # noqa: E402

NAMES = sorted(G.CASES)


def load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz")) as z:  # no pickles
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", NAMES)
def test_golden_inputs_regenerate(name):
    f = load(name)
    packed, scales, x = G.inputs(name)
    assert np.array_equal(packed, f["packed"]) and np.array_equal(scales, f["scales"]) and np.array_equal(x, f["x"])


@pytest.mark.parametrize("name", NAMES)
def test_golden_oracle_outputs(name):
    f = load(name)
    out = G.outputs(name, f["packed"], f["scales"], f["x"])
    for key, v in out.items():
        assert np.array_equal(v, f[key]), key


@pytest.mark.parametrize("name", NAMES)
def test_golden_within_reference_bound(name):
    f = load(name)
    _, _, bits, n, k, g = G.CASES[name]
    ref = f["ref64"].reshape(G.M, n)
    mag = f["mag64"].reshape(G.M, n)
    for kind in ("exact", "default"):
        y = f[f"y_{kind}_m{G.M}"].reshape(G.M, n)
        assert L.max_ulp_bound(y, ref, mag) <= 1.0, kind
        assert L.max_rel_excess(y, ref) <= 2e-3, kind
        y1 = f[f"y_{kind}_m1"].reshape(1, n)
        assert np.array_equal(y1, y[:1]), kind  # row 0 of the batch is the one-token result, bit for bit


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_golden_gpu(name):
    f = load(name)
    _, _, bits, n, k, g = G.CASES[name]
    K = L.kernels()
    lin = L.Linear(f["packed"], f["scales"], n, k, g, bits)
    L.check(lin.rc, "repack")
    wt, st = lin.host_kt()
    assert np.array_equal(wt, f["wt"]) and np.array_equal(st, f["st"])
    w = L.Dev(8 * k * 2)
    L.check(K.ak_wq_dequant_kt_rows(bits, lin.wt.p, lin.st.p, w.p, n, k, g, n - 8, 8, None), "dequant")
    assert np.array_equal(w.get(np.uint16, 8 * k), f["deq_last8"])
    try:
        for mode, kind in ((1, "default"), (0, "exact")):
            L.check(K.ak_w4_set_mma(mode), "ak_w4_set_mma")
            for m in (1, G.M):
                xd = L.Dev.of(f["x"][: m * k])
                (y,) = L.gemv(bits, xd, m, [lin], k, g)
                assert np.array_equal(y.get(np.uint16, m * n), f[f"y_{kind}_m{m}"]), (kind, m)
    finally:
        K.ak_w4_set_mma(-1)
