"""The W4 / W3 convenience entry points (reference: kernels/include/agens_kernels.h:181-248, w4_gemv.cu:585-607,
702-752, 845-848, 897-935, 3263-3270) on the GPU: each one called through the C ABI against the oracle (and against
ak_wq_gemv_kt_multi / ak_wq_repack_kt / ak_wq_dequant_kt_rows, which they forward to).

Shape: 301 rows (a padded last 4- and 16-row block), k = 2304 (a padded last 1024-input tile), group 128 and 64.
"""
import ctypes

import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, ptr_array, int_array, gen_container, gen_scales, gen_x, ora_repack,
                  ora_fast, ora_exact, oracle, ptr)

pytestmark = pytest.mark.gpu

N, KIN = 301, 2304


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


def container(seed, bits, n=N, k=KIN, group=128):
    lo, span = -(1 << (bits - 1)), 1 << bits
    return gen_container(seed, n, k, lo, span), gen_scales(seed + 1, n * k // group)


def dev_out(nbytes):
    return Dev(nbytes)


@pytest.mark.parametrize("group", [128, 64])
def test_repack_conveniences_bytes(group):
    K = kernels()
    for bits, fn in ((4, "ak_w4_repack_kt"), (3, "ak_w3_repack_kt")):
        p, s = container(5000 + bits, bits, group=group)
        P, S = Dev.of(p), Dev.of(s)
        W = Dev(K.ak_wq_kt_weight_bytes(bits, N, KIN))
        T = Dev(K.ak_w4_kt_scale_bytes(N, KIN, group))
        check(getattr(K, fn)(P.p, S.p, W.p, T.p, N, KIN, group, None), fn)
        check(K.ak_synchronize())
        rc, owt, ost = ora_repack(bits, p, s, N, KIN, group)
        assert rc == 0
        assert np.array_equal(W.get(np.uint8, owt.size), owt), fn
        assert np.array_equal(T.get(np.uint16, ost.size), ost), fn
    # the g128 form (agens_kernels.h:183) and its sizes
    p, s = container(5010, 4)
    P, S = Dev.of(p), Dev.of(s)
    W = Dev(K.ak_w4g128_kt_weight_bytes(N, KIN))
    T = Dev(K.ak_w4g128_kt_scale_bytes(N, KIN))
    check(K.ak_w4g128_repack_kt(P.p, S.p, W.p, T.p, N, KIN, None), "ak_w4g128_repack_kt")
    check(K.ak_synchronize())
    rc, owt, ost = ora_repack(4, p, s, N, KIN, 128)
    assert np.array_equal(W.get(np.uint8, owt.size), owt) and np.array_equal(T.get(np.uint16, ost.size), ost)


@pytest.mark.parametrize("group", [128, 64])
def test_dequant_conveniences(group):
    K = kernels()
    for bits in (4, 3):
        p, s = container(5020 + bits, bits, group=group)
        L = Linear(p, s, N, KIN, group, bits)
        check(L.rc)
        wt, st = L.host_kt()
        for r0, nr in ((0, N), (37, 100)):
            ref = np.zeros(nr * KIN, dtype=np.uint16)
            assert oracle().ora_dequant_kt_rows(bits, ptr(wt), ptr(st), ptr(ref), N, KIN, group, r0, nr) == 0
            Wd = Dev(nr * KIN * 2)
            if bits == 4:
                if r0 == 0 and nr == N:
                    check(K.ak_w4_dequant_kt(L.wt.p, L.st.p, Wd.p, N, KIN, group, None), "ak_w4_dequant_kt")
                else:
                    check(K.ak_w4_dequant_kt_rows(L.wt.p, L.st.p, Wd.p, N, KIN, group, r0, nr, None), "w4 rows")
            else:
                check(K.ak_w3_dequant_kt_rows(L.wt.p, L.st.p, Wd.p, N, KIN, group, r0, nr, None), "w3 rows")
            assert np.array_equal(Wd.get(np.uint16, nr * KIN), ref), (bits, r0, nr)


@pytest.mark.parametrize("group", [128, 64])
@pytest.mark.parametrize("mode", [1, 0])
def test_gemv_conveniences(group, mode):
    """ak_w4_gemv_kt / _multi / _batched (bf16w 0 and 1), ak_w3_gemv_kt / _multi / _batched, ak_w4_mma_gemv, under
    both numerics switches (ak_w4_mma_gemv always takes the default numerics)."""
    K = kernels()
    K.ak_w4_set_mma(mode)
    ora = ora_fast if mode == 1 else ora_exact
    try:
        for bits in (4, 3):
            segs = []
            for i, n in enumerate((N, 128, 64)):
                p, s = container(5100 + 10 * bits + i, bits, n=n, group=group)
                L = Linear(p, s, n, KIN, group, bits)
                check(L.rc)
                segs.append((L,) + L.host_kt())
            x = gen_x(5200 + bits, 5 * KIN)
            X = Dev.of(x)
            L, wt, st = segs[0]
            # m = 1
            Y = Dev(N * 2)
            if bits == 4:
                check(K.ak_w4_gemv_kt(X.p, L.wt.p, L.st.p, Y.p, N, KIN, group, 0, None), "ak_w4_gemv_kt")
            else:
                check(K.ak_w3_gemv_kt(X.p, L.wt.p, L.st.p, Y.p, N, KIN, group, None), "ak_w3_gemv_kt")
            assert np.array_equal(Y.get(np.uint16, N), ora(bits, x, 1, wt, st, N, KIN, group)[0])
            # batched, 5 tokens
            Yb = Dev(5 * N * 2)
            if bits == 4:
                check(K.ak_w4_gemv_kt_batched(X.p, L.wt.p, L.st.p, Yb.p, 5, N, KIN, group, 0, None), "w4 batched")
            else:
                check(K.ak_w3_gemv_kt_batched(X.p, L.wt.p, L.st.p, Yb.p, 5, N, KIN, group, None), "w3 batched")
            assert np.array_equal(Yb.get(np.uint16, 5 * N).reshape(5, N), ora(bits, x, 5, wt, st, N, KIN, group))
            # multi: three segments of one launch
            ys = [Dev(l.n * 2) for l, _, _ in segs]
            wts = ptr_array([l.wt.p for l, _, _ in segs])
            sts = ptr_array([l.st.p for l, _, _ in segs])
            yp = ptr_array([y.p for y in ys])
            ns = int_array([l.n for l, _, _ in segs])
            if bits == 4:
                check(K.ak_w4_gemv_kt_multi(X.p, 3, wts, sts, yp, ns, KIN, group, 0, None), "w4 multi")
            else:
                check(K.ak_w3_gemv_kt_multi(X.p, 3, wts, sts, yp, ns, KIN, group, None), "w3 multi")
            for (l, w, s), y in zip(segs, ys):
                assert np.array_equal(y.get(np.uint16, l.n), ora(bits, x, 1, w, s, l.n, KIN, group)[0])
            if bits == 4:
                # bf16w = 1: weights rounded to bf16(q * s) first, on the fp32 path whatever the switch
                check(K.ak_w4_gemv_kt(X.p, L.wt.p, L.st.p, Y.p, N, KIN, group, 1, None), "w4 bf16w")
                assert np.array_equal(Y.get(np.uint16, N), ora_exact(4, x, 1, wt, st, N, KIN, group, bf16w=1)[0])
                check(K.ak_w4_gemv_kt_batched(X.p, L.wt.p, L.st.p, Yb.p, 5, N, KIN, group, 1, None), "w4 b bf16w")
                assert np.array_equal(Yb.get(np.uint16, 5 * N).reshape(5, N),
                                      ora_exact(4, x, 5, wt, st, N, KIN, group, bf16w=1))
                check(K.ak_w4_gemv_kt_multi(X.p, 3, wts, sts, yp, ns, KIN, group, 1, None), "w4 multi bf16w")
                for (l, w, s), y in zip(segs, ys):
                    assert np.array_equal(y.get(np.uint16, l.n), ora_exact(4, x, 1, w, s, l.n, KIN, group, bf16w=1)[0])
                # the tensor-core entry point: the default numerics at any switch setting
                check(K.ak_w4_mma_gemv(X.p, L.wt.p, L.st.p, Yb.p, 5, N, KIN, group, None), "ak_w4_mma_gemv")
                assert np.array_equal(Yb.get(np.uint16, 5 * N).reshape(5, N), ora_fast(4, x, 5, wt, st, N, KIN, group))
    finally:
        K.ak_w4_set_mma(1)


def test_w4g128_kt_bf16():
    """ak_w4g128_gemv_kt_bf16 (agens_kernels.h:184): the g128 KT GEMV of the reference's exact fp32 order."""
    K = kernels()
    p, s = container(5300, 4)
    L = Linear(p, s, N, KIN, 128, 4)
    check(L.rc)
    wt, st = L.host_kt()
    x = gen_x(5301, KIN)
    X = Dev.of(x)
    Y = Dev(N * 2)
    check(K.ak_w4g128_gemv_kt_bf16(X.p, L.wt.p, L.st.p, Y.p, N, KIN, None), "ak_w4g128_gemv_kt_bf16")
    assert np.array_equal(Y.get(np.uint16, N), ora_exact(4, x, 1, wt, st, N, KIN, 128)[0])
