"""ak_wq_gemv_kt_multi_noalloc (include/agens_kernels.h; no counterpart in the reference): the GEMV entry point that
allocates nothing, its split-K partials and counters in the library's static device array.

Bar: bit-identical to ak_wq_gemv_kt_multi on the same inputs, on two calls in a row (the second with a smaller
input: fewer tokens and rows, so stale partials or counters of the first call would show), at shapes whose routes use
split-K scratch (long k at 1 and 4 tokens, few rows per CU at 8 tokens, both 8-token halves of 16 tokens at long k);
free device memory unchanged by the calls after the first one on the device (its set-up); a call whose worst-case scratch exceeds the array is refused (1)
before any launch.
"""
import ctypes

import numpy as np
import pytest

from _lib import kernels, check, Dev, Linear, ptr_array, int_array, gen_container, gen_scales, gen_x

pytestmark = pytest.mark.gpu


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


def lin(seed, n, k, bits):
    lo, span = -(1 << (bits - 1)), 1 << bits
    L = Linear(gen_container(seed, n, k, lo, span), gen_scales(seed + 1, n * k // 128), n, k, 128, bits)
    check(L.rc)
    return L


def call(fn, bits, X, m, lins, k, ys, ldy=None):
    K = kernels()
    return getattr(K, fn)(bits, X.p, m, len(lins), ptr_array([L.wt.p for L in lins]),
                          ptr_array([L.st.p for L in lins]), ptr_array([y.p for y in ys]),
                          int_array([L.n for L in lins]), int_array(ldy) if ldy else None, k, 128, 0, None)


def free_mem():
    K = kernels()
    f, t = ctypes.c_size_t(), ctypes.c_size_t()
    check(K.ak_mem_info(ctypes.byref(f), ctypes.byref(t)))
    return f.value


# (bits, segment rows, k, first m, second m, rows of the second call)
CASES = [(2, [5120], 27648, 1, 1, [4096]),            # split-K, 1 token (line-load kernel)
         (3, [5120], 27648, 4, 2, [1000]),            # split-K, tokens in A rows
         (4, [5120, 1024, 1024], 5120, 8, 3, [2048, 512, 512]),  # few rows per CU: split-K over 3 segments
         (2, [5120], 27648, 16, 9, [3000])]           # both 8-token halves in one split-K launch


@pytest.mark.parametrize("bits,ns,k,m1,m2,ns2", CASES)
def test_noalloc_matches_gemv_two_calls(bits, ns, k, m1, m2, ns2):
    K = kernels()
    lins = [lin(9000 + 10 * i + bits, n, k, bits) for i, n in enumerate(ns)]
    x = gen_x(9100 + m1, m1 * k)
    X = Dev.of(x)
    # first call: every output of the reference entry point, then the no-alloc one into separate buffers
    ref = [Dev(m1 * L.n * 2) for L in lins]
    check(call("ak_wq_gemv_kt_multi", bits, X, m1, lins, k, ref), "gemv")
    check(K.ak_synchronize())
    want1 = [y.get(np.uint16, m1 * L.n) for y, L in zip(ref, lins)]
    got = [Dev(m1 * L.n * 2) for L in lins]
    check(call("ak_wq_gemv_kt_multi_noalloc", bits, X, m1, lins, k, got), "noalloc")
    check(K.ak_synchronize())
    for i, (y, L) in enumerate(zip(got, lins)):
        assert np.array_equal(y.get(np.uint16, m1 * L.n), want1[i]), f"first call, segment {i}"
    # second call: fewer tokens and rows (the first rows of each segment: same weights, n smaller), new x
    x2 = gen_x(9200 + m2, m2 * k)
    X2 = Dev.of(x2)
    small = []
    for L, n2 in zip(lins, ns2):
        S = Linear.__new__(Linear)
        S.n, S.k, S.group, S.bits, S.wt, S.st = n2, k, 128, bits, L.wt, L.st
        small.append(S)
    # rows [0, n2) of an n-row KT are not an n2-row KT (records are (t * n + o)): compare against the reference
    # entry point on the same arguments instead of against the first call
    ref2 = [Dev(m2 * S.n * 2) for S in small]
    got2 = [Dev(m2 * S.n * 2) for S in small]
    # after the first call on the device (its set-up: the runtime places the static array when the symbol's address
    # is first taken), further calls leave the free device memory as it is (every buffer of the test is allocated)
    check(K.ak_synchronize())
    before = free_mem()
    check(call("ak_wq_gemv_kt_multi_noalloc", bits, X2, m2, small, k, got2), "noalloc 2")
    check(K.ak_synchronize())
    mid = free_mem()
    check(call("ak_wq_gemv_kt_multi", bits, X2, m2, small, k, ref2), "gemv 2")
    check(K.ak_synchronize())
    for i, (a, b, S) in enumerate(zip(got2, ref2, small)):
        assert np.array_equal(a.get(np.uint16, m2 * S.n), b.get(np.uint16, m2 * S.n)), f"second call, segment {i}"
    assert mid == before, "the no-alloc entry point changed the free device memory"


def scratch_need(m, ns, k):
    """noalloc_scratch_need of wq_api.hip: 4096 + 64 * P * T * sum(ceil(n / 16))."""
    P = min(8, (k + 1023) // 1024)
    mm = min(m, 16)
    T = 4 if mm <= 4 else 8 if mm <= 8 else 16
    return 4096 + 64 * P * T * sum((n + 15) // 16 for n in ns)


def test_noalloc_refuses_beyond_its_scratch():
    """A call whose worst-case scratch exceeds the 64 MiB array returns 1 before anything is launched.  The buffers
    are real and large enough for the call, so that a wrong acceptance would run an in-bounds launch."""
    K = kernels()
    n, k, m = 140000, 8192, 16
    assert scratch_need(m, [n], k) > 64 << 20
    assert scratch_need(8, [n], k) <= 64 << 20
    W = Dev(K.ak_wq_kt_weight_bytes(4, n, k))
    S = Dev(K.ak_w4_kt_scale_bytes(n, k, 128))
    X, Y = Dev(m * k * 2), Dev(m * n * 2)
    rc = K.ak_wq_gemv_kt_multi_noalloc(4, X.p, m, 1, ptr_array([W.p]), ptr_array([S.p]), ptr_array([Y.p]),
                                        int_array([n]), None, k, 128, 0, None)
    assert rc == 1
    check(K.ak_synchronize())
