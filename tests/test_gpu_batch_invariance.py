"""Batch invariance under the library's DEFAULT routing (no ak_wq_set_mm_min override anywhere in this module).

The reference's contract for batched launches: every row of an m-token launch is bit-identical to the same token's
row from launches of at most 8 tokens (kernels/src/w4_gemv.cu:1075-1079), and to the m = 1 GEMV
(kernels/bench/test_w4.cu:143-158).  With the default routing, 17..128 tokens at k <= 8192 take the fp16-MFMA kernel
(csrc/wq_mm.hip) and at most 8 the integer-limb kernels: these tests check that both give the same bits.

- test_batched_rows_equal_8_token_launches: kernels/bench/test_wq.cu:265-297 restated (bits 2 / 3 / 4, group 64 and
  128, shapes 5120 x 6144, 1280 x 5120, 301 x 1152, m = 72, 37, 13 against 8-token launches; x uniform in [-1, 1));
- test_batched_rows_equal_single_token: kernels/bench/test_w4.cu:143-158 (ak_w4_gemv_kt_batched, m = 2..16 against
  the m = 1 GEMV), plus m = 24, 40 and 128;
- the default route against the oracle (ora_gemv_fast_kt) bit for bit, through ak_wq_gemv_kt_multi, the no-alloc
  entry point (16 and 64 tokens) and the W4 / W3 conveniences at m >= 9.
"""
import ctypes

import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, gemv, gen_container, gen_scales, gen_x, f2bf_array, ora_repack,
                  ora_fast, ptr_array, int_array)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    # the library's defaults: the default numerics and the default crossover (another module may have left a switch)
    K.ak_w4_set_mma(-1)
    K.ak_wq_set_mm_min(-1)
    yield K


def lin(seed, n, k, bits, group):
    lo, span = -(1 << (bits - 1)), 1 << bits
    L = Linear(gen_container(seed, n, k, lo, span), gen_scales(seed + 1, n * k // group), n, k, group, bits)
    check(L.rc, "repack")
    return L


def uniform_x(seed, count):
    """bf16 of uniform [-1, 1) values (test_wq.cu:275)."""
    return f2bf_array(np.random.default_rng(seed).uniform(-1.0, 1.0, count).astype(np.float32))


def multi(bits, X, m, L, Y, k, group, x_off=0, y_off=0):
    K = kernels()
    rc = K.ak_wq_gemv_kt_multi(bits, X.addr(x_off), m, 1, ptr_array([L.wt.p]), ptr_array([L.st.p]),
                               ptr_array([Y.addr(y_off)]), int_array([L.n]), None, k, group, 0, None)
    check(rc, "ak_wq_gemv_kt_multi")


SHAPES = [(5120, 6144), (1280, 5120), (301, 1152)]


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("n,k", SHAPES)
def test_batched_rows_equal_8_token_launches(bits, group, n, k):
    K = kernels()
    L = lin(7100 + bits * 10 + group + n % 97, n, k, bits, group)
    MB = 72
    X = Dev.of(uniform_x(7200 + bits + n, MB * k))
    Ya, Yb = Dev(MB * n * 2), Dev(MB * n * 2)
    for m in (72, 37, 13):
        multi(bits, X, m, L, Ya, k, group)
        for m0 in range(0, m, 8):
            multi(bits, X, min(8, m - m0), L, Yb, k, group, x_off=m0 * k * 2, y_off=m0 * n * 2)
        check(K.ak_synchronize())
        a, b = Ya.get(np.uint16, m * n), Yb.get(np.uint16, m * n)
        if not np.array_equal(a, b):
            bad = np.argwhere(a.reshape(m, n) != b.reshape(m, n))[:4]
            raise AssertionError(f"W{bits} g{group} {n}x{k} m={m}: {int(np.sum(a != b))} outputs differ from 8-token "
                                 f"launches, e.g. (token, row) {bad.tolist()}")


@pytest.mark.parametrize("n,k,group", [(5120, 5120, 128), (1000, 3072, 64), (7168, 5120, 128)])
def test_batched_rows_equal_single_token(n, k, group):
    K = kernels()
    L = lin(7300 + n % 89, n, k, 4, group)
    M = 128
    x = gen_x(7301 + n, M * k)
    X, Y = Dev.of(x), Dev(M * n * 2)
    y1 = np.zeros((M, n), dtype=np.uint16)
    for i in range(M):  # every token alone (the m = 1 GEMV)
        check(K.ak_w4_gemv_kt(X.addr(i * k * 2), L.wt.p, L.st.p, Y.addr(i * n * 2), n, k, group, 0, None), "gemv")
    check(K.ak_synchronize())
    y1[:] = Y.get(np.uint16, M * n).reshape(M, n)
    for m in list(range(2, 17)) + [24, 40, 128]:
        check(K.ak_w4_gemv_kt_batched(X.p, L.wt.p, L.st.p, Y.p, m, n, k, group, 0, None), "batched")
        check(K.ak_synchronize())
        yb = Y.get(np.uint16, m * n).reshape(m, n)
        assert np.array_equal(yb, y1[:m]), f"m={m}: {int(np.sum(yb != y1[:m]))} outputs differ from the m = 1 GEMV"


def oracle_rows(L, bits, x, m, r0, r1):
    words, sg = L.k // 8, L.k // L.group
    p = np.ascontiguousarray(L.packed[r0 * words:r1 * words])
    s = np.ascontiguousarray(L.scales[r0 * sg:r1 * sg])
    rc, wt, st = ora_repack(bits, p, s, r1 - r0, L.k, L.group)
    assert rc == 0
    return ora_fast(bits, x, m, wt, st, r1 - r0, L.k, L.group)


def assert_oracle(y, L, bits, x, m, what):
    for r0 in sorted({0, max(0, L.n // 2 - 32), max(0, L.n - 64)}):
        r1 = min(L.n, r0 + 64)
        want = oracle_rows(L, bits, x, m, r0, r1)
        got = np.ascontiguousarray(y[:, r0:r1])
        assert np.array_equal(got, want), f"{what}: rows {r0}..{r1}: {int(np.sum(got != want))} outputs differ"


@pytest.mark.parametrize("bits,n,k,m", [(3, 55296, 5120, 16), (2, 5120, 27648, 16), (4, 7168, 5120, 40),
                                        (3, 5120, 5120, 128), (2, 1000, 2048, 9), (2, 55296, 5120, 2)])
def test_default_route_against_oracle(bits, n, k, m):
    L = lin(7400 + bits + m, n, k, bits, 128)
    x = gen_x(7401 + m, m * k, 0.5 if k > 8192 else 1.0)
    (Y,) = gemv(bits, Dev.of(x), m, [L], k, 128)
    assert_oracle(Y.get(np.uint16, m * n).reshape(m, n), L, bits, x, m, f"W{bits} {n}x{k} m={m}")


@pytest.mark.parametrize("m", [16, 64])
def test_noalloc_default_route(m):
    """The no-alloc entry point at 16 and 64 tokens on the default route (few rows per CU: the MFMA route's split-K
    partials in the static array), bit-identical to ak_wq_gemv_kt_multi and to the oracle, on two calls in a row."""
    K = kernels()
    k = 5120
    lins = [lin(7500 + i, n, k, 4, 128) for i, n in enumerate((5120, 1024, 1024))]
    for call, mm in enumerate((m, m // 2 + 1)):
        x = gen_x(7510 + call + m, mm * k)
        X = Dev.of(x)
        outs = {}
        for fn in ("ak_wq_gemv_kt_multi_noalloc", "ak_wq_gemv_kt_multi"):
            ys = [Dev(mm * L.n * 2) for L in lins]
            rc = getattr(K, fn)(4, X.p, mm, 3, ptr_array([L.wt.p for L in lins]), ptr_array([L.st.p for L in lins]),
                                ptr_array([y.p for y in ys]), int_array([L.n for L in lins]), None, k, 128, 0, None)
            check(rc, fn)
            check(K.ak_synchronize())
            outs[fn] = [y.get(np.uint16, mm * L.n).reshape(mm, L.n) for y, L in zip(ys, lins)]
        for i, L in enumerate(lins):
            assert np.array_equal(outs["ak_wq_gemv_kt_multi_noalloc"][i], outs["ak_wq_gemv_kt_multi"][i])
            assert_oracle(outs["ak_wq_gemv_kt_multi"][i], L, 4, x, mm, f"call {call} segment {i} m={mm}")


def test_conveniences_default_route():
    """ak_w4_gemv_kt_batched, ak_w3_gemv_kt_batched and ak_w4_mma_gemv at 9..128 tokens: the oracle's bits."""
    K = kernels()
    k = 3072
    L4, L3 = lin(7600, 700, k, 4, 128), lin(7601, 700, k, 3, 128)
    for m in (9, 24, 100):
        x = gen_x(7610 + m, m * k)
        X, Y = Dev.of(x), Dev(m * 700 * 2)
        check(K.ak_w4_gemv_kt_batched(X.p, L4.wt.p, L4.st.p, Y.p, m, 700, k, 128, 0, None), "w4 batched")
        check(K.ak_synchronize())
        assert_oracle(Y.get(np.uint16, m * 700).reshape(m, 700), L4, 4, x, m, f"w4 batched m={m}")
        check(K.ak_w3_gemv_kt_batched(X.p, L3.wt.p, L3.st.p, Y.p, m, 700, k, 128, None), "w3 batched")
        check(K.ak_synchronize())
        assert_oracle(Y.get(np.uint16, m * 700).reshape(m, 700), L3, 3, x, m, f"w3 batched m={m}")
        check(K.ak_w4_mma_gemv(X.p, L4.wt.p, L4.st.p, Y.p, m, 700, k, 128, None), "w4 mma")
        check(K.ak_synchronize())
        assert_oracle(Y.get(np.uint16, m * 700).reshape(m, 700), L4, 4, x, m, f"w4 mma m={m}")


@pytest.mark.parametrize("bits", [2, 3])
def test_two_tokens_on_wide_linears_equal_single_token(bits):
    """Two tokens on a wide linear (gate_up 55296 x 5120; W2 takes the tokens-in-A-rows kernel there, W3 the line-load
    kernel): each token's row bit-identical to its one-token launch (kernels/bench/test_w4.cu:143-158)."""
    K = kernels()
    n, k = 55296, 5120
    L = lin(7700 + bits, n, k, bits, 128)
    x = gen_x(7710 + bits, 2 * k)
    X, Y2, Y1 = Dev.of(x), Dev(2 * n * 2), Dev(2 * n * 2)
    multi(bits, X, 2, L, Y2, k, 128)
    for t in range(2):
        multi(bits, X, 1, L, Y1, k, 128, x_off=t * k * 2, y_off=t * n * 2)
    check(K.ak_synchronize())
    a, b = Y2.get(np.uint16, 2 * n), Y1.get(np.uint16, 2 * n)
    assert np.array_equal(a, b), f"W{bits}: {int(np.sum(a != b))} outputs of the 2-token launch differ"
