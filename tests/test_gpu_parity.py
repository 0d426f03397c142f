"""Parity of the HIP path (called through the C ABI) with the CPU oracle, on the GPU.

Bit-exact: repack bytes, dequant, both GEMV numerics.  Within tolerance: the default numerics vs the reference's fp32
CPU path (reference.rs:53-71) and vs fp64 with the reference gate's bound (test_w4.cu:123-141).  Invariants of the
reference gates (test_w4.cu, test_wq.cu): rows bit-identical for any m, multi-segment == separate launches, ldy parts,
W2 / W3 == W4 on the same values, CT == KT, range refusal.
"""
import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, gemv, ptr_array, int_array, gen_container, gen_scales, gen_x,
                  XorShift, f2bf_array, bf2f_array, ora_repack, ora_fast, ora_exact, ora_ref_f32, ora_ref_f64,
                  oracle, ptr, max_rel, max_rel_excess, max_ulp_bound)

pytestmark = pytest.mark.gpu


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
    K.ak_w4_set_lean(0)


def make_linear(seed, n, k, group, bits, lo=None, span=None):
    lo = -(1 << (bits - 1)) if lo is None else lo
    span = (1 << bits) if span is None else span
    packed = gen_container(seed, n, k, lo, span)
    scales = gen_scales(seed + 1, n * k // group)
    return Linear(packed, scales, n, k, group, bits)


def y_of(ys, m, n, ldy=None):
    return ys.get(np.uint16, m * (ldy or n)).reshape(m, ldy or n)


SHAPES = [(256, 5120), (77, 640), (301, 1152), (1024, 2048), (96, 3072)]


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("group", [128, 64])
@pytest.mark.parametrize("n,k", SHAPES)
def test_repack_bytes_and_dequant(bits, group, n, k):
    if k % group:
        pytest.skip("k % group")
    L = make_linear(100 + bits, n, k, group, bits)
    assert L.rc == 0
    wt, st = L.host_kt()
    rc, owt, ost = ora_repack(bits, L.packed, L.scales, n, k, group)
    assert rc == 0
    assert (wt == owt).all() and (st == ost).all()
    K = kernels()
    for r0, nr in ((0, n), (n // 3, max(1, n // 2))):
        W = Dev(nr * k * 2)
        check(K.ak_wq_dequant_kt_rows(bits, L.wt.p, L.st.p, W.p, n, k, group, r0, nr, None))
        got = W.get(np.uint16, nr * k)
        ref = np.zeros(nr * k, dtype=np.uint16)
        assert oracle().ora_dequant_kt_rows(bits, ptr(owt), ptr(ost), ptr(ref), n, k, group, r0, nr) == 0
        assert (got == ref).all()


def test_repack_range_codes():
    # test_wq.cu:249-269
    K = kernels()
    n, k, g = 64, 1024, 64
    w3 = make_linear(1, n, k, g, 3)
    assert w3.rc == 0
    W2 = Dev(K.ak_wq_kt_weight_bytes(2, n, k))
    S2 = Dev(K.ak_w4_kt_scale_bytes(n, k, g))
    assert K.ak_wq_repack_kt(2, w3.P.p, w3.S.p, W2.p, S2.p, n, k, g, None) == 1
    w4 = make_linear(2, n, k, g, 4)
    W3 = Dev(K.ak_wq_kt_weight_bytes(3, n, k))
    assert K.ak_wq_repack_kt(3, w4.P.p, w4.S.p, W3.p, S2.p, n, k, g, None) == 1
    w2 = make_linear(3, n, k, g, 2)
    assert K.ak_wq_repack_kt(3, w2.P.p, w2.S.p, W3.p, S2.p, n, k, g, None) == 0
    check(K.ak_synchronize())


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("group", [128, 64])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 3, 8, 16])
def test_default_gemv_bitexact(bits, group, n, k, m):
    if k % group:
        pytest.skip("k % group")
    L = make_linear(200 + bits, n, k, group, bits)
    x = gen_x(300 + m, m * k)
    X = Dev.of(x)
    (Y,) = gemv(bits, X, m, [L], k, group)
    y = y_of(Y, m, n)
    wt, st = L.host_kt()
    assert (y == ora_fast(bits, x, m, wt, st, n, k, group)).all()
    ref32 = ora_ref_f32(x, m, L.packed, L.scales, n, k, group)
    ref64, mag = ora_ref_f64(x, m, L.packed, L.scales, n, k, group)
    assert max_rel_excess(y, ref32) <= 2e-3
    assert max_ulp_bound(y, ref64, mag) <= 1.0


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("group", [128, 64])
@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("bf16w", [0, 1])
def test_exact_gemv_bitexact(bits, group, m, bf16w):
    K = kernels()
    n, k = 301, 2304 if group == 128 else 1152
    L = make_linear(400 + bits, n, k, group, bits)
    x = gen_x(500 + m, m * k)
    X = Dev.of(x)
    K.ak_w4_set_mma(0)
    try:
        (Y,) = gemv(bits, X, m, [L], k, group, bf16w=bf16w)
    finally:
        K.ak_w4_set_mma(1)
    y = y_of(Y, m, n)
    wt, st = L.host_kt()
    assert (y == ora_exact(bits, x, m, wt, st, n, k, group, bf16w=bf16w)).all()
    if not bf16w:  # bf16w goes to the exact path whatever the mode
        (Y2,) = gemv(bits, X, m, [L], k, group, bf16w=0)
        assert (y_of(Y2, m, n) == ora_fast(bits, x, m, wt, st, n, k, group)).all()


@pytest.mark.parametrize("mode", [1, 0])
def test_rows_identical_for_any_m(mode):
    # test_w4.cu:143-158: batched rows == m = 1 rows, both numerics
    K = kernels()
    n, k, g = 1000, 5120, 128
    L = make_linear(600, n, k, g, 4)
    x = gen_x(601, 16 * k)
    X = Dev.of(x)
    K.ak_w4_set_mma(mode)
    try:
        ones = [y_of(gemv(4, X.addr(j * k * 2), 1, [L], k, g)[0], 1, n)[0] for j in range(16)]
        for m in (2, 5, 9, 16):
            y = y_of(gemv(4, X, m, [L], k, g)[0], m, n)
            for j in range(m):
                assert (y[j] == ones[j]).all()
    finally:
        K.ak_w4_set_mma(1)


@pytest.mark.parametrize("bits", [4, 3])
def test_multi_segment_and_ldy_parts(bits):
    # test_w4.cu:231-271, test_wq.cu:220-240
    n, k, g = 900, 3072, 128
    n0, n1, n2 = 300, 300, 300
    parts = [make_linear(700 + i, ni, k, g, bits) for i, ni in enumerate((n0, n1, n2))]
    for m in (1, 8):
        x = gen_x(710 + m, m * k)
        X = Dev.of(x)
        ys = gemv(bits, X, m, parts, k, g)
        for i, L in enumerate(parts):
            (Ys,) = gemv(bits, X, m, [L], k, g)
            assert (y_of(ys[i], m, L.n) == y_of(Ys, m, L.n)).all()
        # two parts into one output of row stride n0 + n1 (gate / up of different types)
        ld = n0 + n1
        Y = Dev(m * ld * 2)
        gemv(bits, X, m, [parts[0]], k, g, ldy=[ld], ys=[Y.p])
        gemv(bits, X, m, [parts[1]], k, g, ldy=[ld], ys=[Y.addr(n0 * 2)])
        y = y_of(Y, m, ld)
        assert (y[:, :n0] == y_of(ys[0], m, n0)).all()
        assert (y[:, n0:] == y_of(ys[1], m, n1)).all()


@pytest.mark.parametrize("bits", [3, 2])
@pytest.mark.parametrize("group", [128, 64])
def test_wq_equals_w4_on_gpu(bits, group):
    # test_wq.cu: W{bits} KT output == W4 KT output on the same values, both numerics, m = 1 / 7
    K = kernels()
    n, k = 512, 6144
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed = gen_container(800 + bits, n, k, lo, span)
    scales = gen_scales(801, n * k // group)
    L4 = Linear(packed, scales, n, k, group, 4)
    Lb = Linear(packed, scales, n, k, group, bits)
    for mode in (1, 0):
        K.ak_w4_set_mma(mode)
        try:
            for m in (1, 7):
                X = Dev.of(gen_x(810 + m, m * k))
                a = y_of(gemv(4, X, m, [L4], k, group)[0], m, n)
                b = y_of(gemv(bits, X, m, [Lb], k, group)[0], m, n)
                assert (a == b).all()
        finally:
            K.ak_w4_set_mma(1)


def test_container_kernel_equals_kt_exact():
    # test_w4.cu section 1: the legacy int4-container GEMV == KT exact path == every tuning variant, bitwise
    K = kernels()
    n, k = 1024, 5120
    L = make_linear(900, n, k, 128, 4)
    x = gen_x(901, k)
    X = Dev.of(x)
    Y = Dev(n * 2)
    check(K.ak_w4g128_gemv_bf16(X.p, L.P.p, L.S.p, Y.p, n, k, None))
    ct = Y.get(np.uint16, n)
    wt, st = L.host_kt()
    assert (ct == ora_exact(4, x, 1, wt, st, n, k, 128)[0]).all()
    for v in (11, 12, 21, 22, 41):
        check(K.ak_w4g128_gemv_kt_variant(v, X.p, L.wt.p, L.st.p, Y.p, n, k, None))
        assert (Y.get(np.uint16, n) == ct).all()
    for v in (11, 12, 14, 21, 22, 41, 42):
        check(K.ak_w4g128_gemv_bf16_variant(v, X.p, L.P.p, L.S.p, Y.p, n, k, None))
        assert (Y.get(np.uint16, n) == ct).all()


def test_large_m_is_chunked_identically():
    # m > 16: rows bit-identical to 8-row launches (test_wq.cu:265-297), both numerics
    K = kernels()
    n, k, g = 512, 2048, 128
    L = make_linear(950, n, k, g, 3)
    x = gen_x(951, 72 * k)
    X = Dev.of(x)
    for mode in (1, 0):
        K.ak_w4_set_mma(mode)
        try:
            for m in (72, 37, 13):
                big = y_of(gemv(3, X, m, [L], k, g)[0], m, n)
                for m0 in range(0, m, 8):
                    mm = min(8, m - m0)
                    part = y_of(gemv(3, X.addr(m0 * k * 2), mm, [L], k, g)[0], mm, n)
                    assert (big[m0:m0 + mm] == part).all()
        finally:
            K.ak_w4_set_mma(1)


def test_long_k_mixed_tokens():
    # long k (down projection) at every token count of one launch: rows equal the oracle and the m = 1 launches
    K = kernels()
    n, k, g = 700, 27648, 128
    L = make_linear(960, n, k, g, 2)
    x = gen_x(961, 12 * k)
    X = Dev.of(x)
    y = y_of(gemv(2, X, 12, [L], k, g)[0], 12, n)
    wt, st = L.host_kt()
    for r0 in (0, n - 64):
        yo = ora_fast(2, x, 12, wt, st, n, k, g, rows=(r0, r0 + 64))
        assert (y[:, r0:r0 + 64] == yo[:, r0:r0 + 64]).all()
    for j in (0, 5, 11):
        one = y_of(gemv(2, X.addr(j * k * 2), 1, [L], k, g)[0], 1, n)[0]
        assert (one == y[j]).all()


@pytest.mark.parametrize("cfg", [0, 1, 2])
def test_baseline_config_shapes(cfg):
    # BASELINE configs 0-2 at full size: bit-exact vs the oracle on sampled row blocks, tolerance vs the fp32
    # reference on the same rows, and run-to-run determinism of the whole output
    bits, n, k, xs, lo, span = {0: (4, 5120, 5120, 1.0, -8, 16), 1: (3, 55296, 5120, 1.0, -4, 8),
                                2: (2, 5120, 27648, 0.5, -2, 4)}[cfg]
    g = 128
    packed = gen_container(1000 + cfg, n, k, lo, span)
    scales = gen_scales(1100 + cfg, n * k // g)
    L = Linear(packed, scales, n, k, g, bits)
    assert L.rc == 0
    x = gen_x(1200 + cfg, k, xs)
    X = Dev.of(x)
    y1 = y_of(gemv(bits, X, 1, [L], k, g)[0], 1, n)
    y2 = y_of(gemv(bits, X, 1, [L], k, g)[0], 1, n)
    assert (y1 == y2).all()
    wt, st = L.host_kt()
    for r0 in (0, n // 2 - 37, n - 64):
        rows = (r0, r0 + 64)
        yo = ora_fast(bits, x, 1, wt, st, n, k, g, rows=rows)
        assert (y1[:, r0:r0 + 64] == yo[:, r0:r0 + 64]).all()
    sub = slice(0, 256)
    p_sub = packed.reshape(n, k // 8)[sub].ravel()
    s_sub = scales.reshape(n, k // g)[sub].ravel()
    ref32 = ora_ref_f32(x, 1, p_sub, s_sub, 256, k, g)
    assert max_rel_excess(y1[:, sub], ref32) <= 2e-3


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8])
def test_long_k_small_m(bits, m):
    """Activations beyond the LDS at 2..8 tokens: one segment (split-K across workgroups, stripe partials added by each
    row range's last workgroup) and two segments (chunks of stripes in one workgroup).  Rows equal the oracle and the
    one-token launches; a second launch repeats the first (the split's counters return to zero)."""
    K = kernels()
    k, g = 27648, 128
    A = make_linear(970 + bits, 900, k, g, bits)
    Bl = make_linear(980 + bits, 136, k, g, bits)
    x = gen_x(990 + m, m * k)
    X = Dev.of(x)
    y1 = y_of(gemv(bits, X, m, [A], k, g)[0], m, 900)
    y1b = y_of(gemv(bits, X, m, [A], k, g)[0], m, 900)
    assert np.array_equal(y1, y1b)
    ya, yb = gemv(bits, X, m, [A, Bl], k, g)
    assert np.array_equal(y_of(ya, m, 900), y1)
    wt, st = A.host_kt()
    wtb, stb = Bl.host_kt()
    for r0 in (0, 448, 900 - 40):
        yo = ora_fast(bits, x, m, wt, st, 900, k, g, rows=(r0, r0 + 40))
        assert (y1[:, r0:r0 + 40] == yo[:, r0:r0 + 40]).all(), f"rows {r0}"
    assert (y_of(yb, m, 136) == ora_fast(bits, x, m, wtb, stb, 136, k, g)).all()
    for j in (0, m - 1):
        one = y_of(gemv(bits, X.addr(j * k * 2), 1, [A], k, g)[0], 1, 900)[0]
        assert (one == y1[j]).all()


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("m", [3, 8, 16])
@pytest.mark.parametrize("k", [2048, 27648])
def test_multi_segment_small_m_oracle(bits, m, k):
    """Unequal segments (a QKV-like 640 / 128 / 128 split) at 3..16 tokens, with an ldy stride on the first: every
    segment equals the oracle (the launch splits k across workgroups, row ranges shared out over the segments)."""
    g = 128
    ns = (640, 128, 128)
    parts = [make_linear(1300 + 10 * bits + i, ni, k, g, bits) for i, ni in enumerate(ns)]
    x = gen_x(1350 + m, m * k)
    X = Dev.of(x)
    ld0 = 700
    ys = [Dev(m * ld0 * 2), Dev(m * ns[1] * 2), Dev(m * ns[2] * 2)]
    for _ in range(2):  # twice: the split's counters return to zero
        gemv(bits, X, m, parts, k, g, ldy=[ld0, ns[1], ns[2]], ys=[y.p for y in ys])
        for i, (L, y) in enumerate(zip(parts, ys)):
            wt, st = L.host_kt()
            got = y_of(y, m, L.n, ld0 if i == 0 else None)[:, :L.n]
            rows = (0, 64) if k > 8192 else None
            want = ora_fast(bits, x, m, wt, st, L.n, k, g, rows=rows)
            if rows:
                got, want = got[:, :64], want[:, :64]
            assert (got == want).all(), f"segment {i}"


def test_exact_order_known_answers_on_gpu():
    """The hand-computed order cases of the oracle tests (EXACT_ORDER_CASES): the GPU exact path gives the reference's
    values, where other summation orders give others; the default numerics give the oracle's (their group sums are
    exact sums of 22-bit fixed-point activations relative to the group's largest: next to 2^24, a 1.0 truncates to 0)."""
    from test_oracle import EXACT_ORDER_CASES
    K = kernels()
    k = 4096
    packed = np.full(k // 8, 0x99999999, dtype=np.uint32)  # q = 1
    scales = np.full(k // 128, 0x3F80, dtype=np.uint16)     # 1.0
    L = Linear(packed, scales, 1, k, 128, 4)
    check(L.rc, "repack")
    for vals, want in EXACT_ORDER_CASES:
        xf = np.zeros(k, dtype=np.float32)
        for i, v in vals.items():
            xf[i] = v
        X = Dev.of(f2bf_array(xf))
        K.ak_w4_set_mma(0)
        try:
            for bw in (0, 1):
                (Y,) = gemv(4, X, 1, [L], k, 128, bf16w=bw)
                assert bf2f_array(Y.get(np.uint16, 1))[0] == want, (vals, bw)
        finally:
            K.ak_w4_set_mma(1)
        (Y,) = gemv(4, X, 1, [L], k, 128)
        wt, st = L.host_kt()
        assert np.array_equal(Y.get(np.uint16, 1), ora_fast(4, f2bf_array(xf), 1, wt, st, 1, k, 128).reshape(-1))


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("m", [9, 12, 16])
def test_long_k_nine_to_sixteen_tokens(bits, m):
    """9..16 tokens at k = 27648, one segment (one stripe's 16-token activation image exceeds the LDS): rows equal
    the oracle, the 8-token launches of the same tokens, and a second launch (the split's counters return to zero)."""
    k, g, n = 27648, 128, 900
    A = make_linear(1970 + bits, n, k, g, bits)
    x = gen_x(1990 + m, m * k)
    X = Dev.of(x)
    y1 = y_of(gemv(bits, X, m, [A], k, g)[0], m, n)
    assert np.array_equal(y1, y_of(gemv(bits, X, m, [A], k, g)[0], m, n))
    lo = y_of(gemv(bits, X, 8, [A], k, g)[0], 8, n)
    hi = y_of(gemv(bits, X.addr(8 * k * 2), m - 8, [A], k, g)[0], m - 8, n)
    assert np.array_equal(y1[:8], lo) and np.array_equal(y1[8:], hi)
    # a strided output (ldy > n): the same rows, the padding columns untouched (token rows 8.. of the second half)
    ld = n + 24
    Ys = Dev.of(np.full(m * ld, 0x7FC1, dtype=np.uint16))
    gemv(bits, X, m, [A], k, g, ldy=[ld], ys=[Ys])
    ys = Ys.get(np.uint16, m * ld).reshape(m, ld)
    assert np.array_equal(ys[:, :n], y1)
    assert (ys[:, n:] == 0x7FC1).all()
    wt, st = A.host_kt()
    for r0 in (0, 448, n - 40):
        yo = ora_fast(bits, x, m, wt, st, n, k, g, rows=(r0, r0 + 40))
        assert (y1[:, r0:r0 + 40] == yo[:, r0:r0 + 40]).all(), f"rows {r0}"
