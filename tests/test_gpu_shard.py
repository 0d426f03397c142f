"""Per-rank shapes of a tensor-parallel 32B decode layer, on one GPU.

The reference shards q/k/v and gate/up by output rows and o_proj / down_proj by k, with one all-reduce of the partial
outputs (crates/agens-core/src/m1.rs:58-77 `tp_rule`, kernels/src/tp_ar.cu:1-17).  Each rank runs the same GEMV at
its shard's shape, so one GPU can show every rank's kernel:

- TP = 2, 4, 8 shard shapes: qkv 7168/T rows (q/k/v segments 5120/T, 1024/T, 1024/T), gate_up 55296/T rows,
  o k = 5120/T, down k = 27648/T.  At TP = 8 down has k = 3456 (27 groups of 128, not a multiple of 1024: the last
  tile is padded) and o has k = 640 (a single, padded tile).
- Row shards: a rank's outputs are bit-identical to the same rows of the unsharded launch (every row's result depends
  only on that row's weights, x and k).
- k shards: every rank's output is bit-identical to the oracle at its shard shape, and the ranks' outputs added in
  fp64 (the all-reduce, which this one-GPU build does not run) are within the sum of their bf16 roundings plus the
  reference's 1e-6 * sum|x*w| of the fp64 product of the whole layer.
"""
import numpy as np
import pytest

from _lib import (kernels, Dev, Linear, gemv, gen_container, gen_scales, gen_x, bf2f_array, ora_fast, ora_ref_f32,
                  ora_ref_f64, max_rel_excess, ulp_bf16)

pytestmark = pytest.mark.gpu

G = 128
LO = {4: -8, 3: -4, 2: -2}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    import ctypes
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    K.ak_w4_set_mma(1)
    K.ak_wq_set_mm_min(0)  # the integer-limb kernels at every m (the same numerics as the MFMA route)
    K.ak_w4_set_lean(0)
    yield K
    K.ak_w4_set_mma(-1)
    K.ak_wq_set_mm_min(-1)


def rows_of(packed, scales, n, k, r0, r1):
    p = packed.reshape(n, k // 8)[r0:r1].ravel().copy()
    s = scales.reshape(n, k // G)[r0:r1].ravel().copy()
    return p, s


def cols_of(packed, scales, n, k, c0, c1):
    p = packed.reshape(n, k // 8)[:, c0 // 8:c1 // 8].ravel().copy()
    s = scales.reshape(n, k // G)[:, c0 // G:c1 // G].ravel().copy()
    return p, s


def y_of(ys, m, n):
    return ys.get(np.uint16, m * n).reshape(m, n)


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("tp", [2, 8])
@pytest.mark.parametrize("m", [1, 4, 16])
def test_row_shards_equal_unsharded_rows(bits, tp, m):
    """gate_up (55296 x 5120) and qkv (q/k/v segments) sharded by rows: each rank's launch on its rows equals the
    unsharded launch's rows, and sampled rows equal the oracle."""
    k = 5120
    n = 55296
    packed = gen_container(7000 + bits, n, k, LO[bits], 1 << bits)
    scales = gen_scales(7100 + bits, n * k // G)
    full = Linear(packed, scales, n, k, G, bits)
    assert full.rc == 0
    x = gen_x(7200 + m, m * k)
    X = Dev.of(x)
    yfull = y_of(gemv(bits, X, m, [full], k, G)[0], m, n)
    ns = n // tp
    for r in (0, tp - 1):
        p, s = rows_of(packed, scales, n, k, r * ns, (r + 1) * ns)
        L = Linear(p, s, ns, k, G, bits)
        assert L.rc == 0
        y = y_of(gemv(bits, X, m, [L], k, G)[0], m, ns)
        assert np.array_equal(y, yfull[:, r * ns:(r + 1) * ns]), f"rank {r}"
        wt, st = L.host_kt()
        for r0 in (0, ns - 48):
            yo = ora_fast(bits, x, m, wt, st, ns, k, G, rows=(r0, r0 + 48))
            assert np.array_equal(y[:, r0:r0 + 48], yo[:, r0:r0 + 48]), f"rank {r} rows {r0}"
    # qkv of one rank: q/k/v segments of 5120/tp, 1024/tp, 1024/tp rows in one launch == the same rows launched alone
    nq, nkv = 5120 // tp, 1024 // tp
    segs = []
    for i, (nn, seed) in enumerate(((nq, 7300), (nkv, 7310), (nkv, 7320))):
        pp = gen_container(seed + bits, nn, k, LO[bits], 1 << bits)
        ss = gen_scales(seed + bits + 1, nn * k // G)
        segs.append(Linear(pp, ss, nn, k, G, bits))
    ys = gemv(bits, X, m, segs, k, G)
    for L, yd in zip(segs, ys):
        alone = y_of(gemv(bits, X, m, [L], k, G)[0], m, L.n)
        got = y_of(yd, m, L.n)
        assert np.array_equal(got, alone)
        wt, st = L.host_kt()
        assert np.array_equal(got, ora_fast(bits, x, m, wt, st, L.n, k, G))


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("tp", [2, 4, 8])
@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("which", ["o", "down"])
def test_k_shards(bits, tp, m, which):
    """o (5120 x 5120) and down (5120 x 27648) sharded by k: every rank's output equals the oracle at the shard shape
    (k = 5120/T or 27648/T; padded last tile where the shard is not a multiple of 1024); the fp64 sum of the ranks'
    outputs is within their bf16 roundings + 1e-6 * sum|x*w| of the whole layer's fp64 product; each rank is within
    2e-3 (beyond its own output rounding) of the reference's fp32 CPU path on sampled rows."""
    n, k = (5120, 5120) if which == "o" else (5120, 27648)
    xs = 1.0 if which == "o" else 0.5
    packed = gen_container(7400 + bits + 10 * tp, n, k, LO[bits], 1 << bits)
    scales = gen_scales(7500 + bits + 10 * tp, n * k // G)
    x = gen_x(7600 + m + tp, m * k, xs)
    xm = x.reshape(m, k)
    ks = k // tp
    rows = slice(0, 256)
    total = np.zeros((m, 256), dtype=np.float64)
    ulps = np.zeros((m, 256), dtype=np.float64)
    for r in range(tp):
        p, s = cols_of(packed, scales, n, k, r * ks, (r + 1) * ks)
        L = Linear(p, s, n, ks, G, bits)
        assert L.rc == 0
        xr = np.ascontiguousarray(xm[:, r * ks:(r + 1) * ks]).ravel()
        Xr = Dev.of(xr)
        y = y_of(gemv(bits, Xr, m, [L], ks, G)[0], m, n)
        wt, st = L.host_kt()
        for r0 in (0, 2500, n - 64):
            yo = ora_fast(bits, xr, m, wt, st, n, ks, G, rows=(r0, r0 + 64))
            assert np.array_equal(y[:, r0:r0 + 64], yo[:, r0:r0 + 64]), f"rank {r} rows {r0}"
        ps, ss = rows_of(p, s, n, ks, 0, 256)
        assert max_rel_excess(y[:, rows], ora_ref_f32(xr, m, ps, ss, 256, ks, G)) <= 2e-3, f"rank {r}"
        yf = bf2f_array(y[:, rows]).astype(np.float64)
        total += yf
        ulps += ulp_bf16(yf)
    pf, sf = rows_of(packed, scales, n, k, 0, 256)
    ref64, mag = ora_ref_f64(x, m, pf, sf, 256, k, G)
    err = np.abs(total - ref64)
    assert np.all(err <= ulps + 1e-6 * mag + 1e-30), float(np.max(err / (ulps + 1e-6 * mag + 1e-30)))
