"""The fused prefill GEMM (ak_wq_gemm_kt: dequantize-in-GEMM from the KT layout, the fusion of ak_wq_dequant_kt_rows
and ak_bf16_linear_f32reduce_ld that the model's linear() runs above 128 tokens, kernels/m1/m1_model.cu:1876-1897) on
the GPU.

Bar: the weights are the oracle's dequantized values (ora_dequant_kt_rows, bf16_rn(q * s), pinned against the
reference's dequant), the products are summed in fp32 in the kernel's order, so the result must lie within one bf16
rounding plus k * 2^-24 * sum |x w| of the fp64 product of the same bf16 values, as the library route's (rocBLAS
gemm_ex) does; both routes are also compared with each other under twice that bound.  Exact on small-integer operands
(every order gives the exact sum: pins the operand layouts, the tiles' edges and the row / token mapping).
"""
import ctypes

import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, gemv, gen_container, gen_scales, gen_x, oracle, ptr, bf2f_array,
                  f2bf_array, ulp_bf16)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    yield K


def make(seed, n, k, group, bits, scale_pow2=False):
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed = gen_container(seed, n, k, lo, span)
    if scale_pow2:  # scales 2^-e: products and sums of small-integer inputs stay exact
        rng = np.random.default_rng(seed)
        scales = f2bf_array(np.ldexp(1.0, -rng.integers(2, 6, n * k // group)).astype(np.float32))
    else:
        scales = gen_scales(seed + 1, n * k // group)
    L = Linear(packed, scales, n, k, group, bits)
    check(L.rc)
    return L


def dequant_host(L, r0=0, nr=None):
    nr = L.n - r0 if nr is None else nr
    wt, st = L.host_kt()
    w = np.zeros(nr * L.k, dtype=np.uint16)
    assert oracle().ora_dequant_kt_rows(L.bits, ptr(wt), ptr(st), ptr(w), L.n, L.k, L.group, r0, nr) == 0
    return w.reshape(nr, L.k)


def gemm(L, X, m, ldy=None, fill=None):
    K = kernels()
    ld = ldy or L.n
    Y = Dev.of(np.full(m * ld, fill, dtype=np.uint16)) if fill is not None else Dev(m * ld * 2)
    check(K.ak_wq_gemm_kt(L.bits, X.p, m, L.wt.p, L.st.p, Y.p, L.n, ldy or 0, L.k, L.group, None), "ak_wq_gemm_kt")
    check(K.ak_synchronize(), "sync")
    return Y.get(np.uint16, m * ld).reshape(m, ld)


def within(y, x, w, k, factor=1.0):
    xf, wf = bf2f_array(x).astype(np.float64), bf2f_array(w).astype(np.float64)
    ref, mag = xf @ wf.T, np.abs(xf) @ np.abs(wf).T
    err = np.abs(bf2f_array(y).astype(np.float64) - ref)
    bound = factor * (ulp_bf16(ref) + mag * k * 2.0 ** -24)
    return float(np.max(err / bound))


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("group", [128, 64])
@pytest.mark.parametrize("m,n,k", [(1, 301, 2304), (129, 77, 640), (200, 300, 1152), (257, 129, 3072)])
def test_gemm_within_fp32_accumulation_bound(bits, group, m, n, k):
    if k % group:
        pytest.skip("k % group")
    L = make(8000 + bits, n, k, group, bits)
    x = gen_x(8100 + m, m * k).reshape(m, k)
    y = gemm(L, Dev.of(x), m)
    assert within(y, x, dequant_host(L), k) <= 1.0


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_gemm_exact_on_small_integer_operands(bits):
    """x in {-3..3} and power-of-two scales: every product and partial sum is exact in fp32, so any summation order
    gives the exact result, bit for bit against the fp64 product (ragged m, n and the ldy stride, padding untouched)."""
    m, n, k, g = 150, 200, 2048, 128
    L = make(8200 + bits, n, k, g, bits, scale_pow2=True)
    rng = np.random.default_rng(8201)
    x = f2bf_array(rng.integers(-3, 4, (m, k)).astype(np.float32))
    ld = n + 40
    y = gemm(L, Dev.of(x), m, ldy=ld, fill=0x7FC1)
    w = dequant_host(L)
    ref = bf2f_array(x).astype(np.float64) @ bf2f_array(w).astype(np.float64).T
    assert np.array_equal(y[:, :n], f2bf_array(ref.astype(np.float32)))
    assert (y[:, n:] == 0x7FC1).all()


@pytest.mark.parametrize("bits", [3, 2])
def test_gemm_prefill_shapes_against_library_route(bits):
    """gate_up-like (n = 4096 of 55296 rows, k = 5120) and down-like (n = 640, k = 27648) at 256 / 512 tokens: within
    the bound of fp64 on sampled rows, and within twice it of the dequantize + rocBLAS route on every output."""
    K = kernels()
    for n, k, m in ((4096, 5120, 512), (640, 27648, 256)):
        L = make(8300 + bits + n, n, k, 128, bits)
        x = gen_x(8400 + m, m * k).reshape(m, k)
        X = Dev.of(x)
        y = gemm(L, X, m)
        W = Dev(n * k * 2)
        check(K.ak_wq_dequant_kt_rows(bits, L.wt.p, L.st.p, W.p, n, k, 128, 0, n, None), "dequant")
        Y2 = Dev(m * n * 2)
        check(K.ak_bf16_linear_f32reduce(X.p, W.p, Y2.p, m, n, k, None), "rocblas")
        check(K.ak_synchronize(), "sync")
        y2 = Y2.get(np.uint16, m * n).reshape(m, n)
        w = W.get(np.uint16, n * k).reshape(n, k)
        rows = np.r_[0:64, n // 2:n // 2 + 64, n - 64:n]
        assert within(y[:, rows], x, w[rows], k) <= 1.0
        a, b = bf2f_array(y).astype(np.float64), bf2f_array(y2).astype(np.float64)
        mag = np.abs(bf2f_array(x).astype(np.float64)) @ np.abs(bf2f_array(w).astype(np.float64)).T
        assert np.all(np.abs(a - b) <= 2 * (ulp_bf16(b) + mag * k * 2.0 ** -24))


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("group", [128, 64])
@pytest.mark.parametrize("m,n,k", [(257, 20557, 640), (520, 14000, 1152)])
def test_gemm_wide_tiles_within_bound(bits, group, m, n, k):
    """Shapes with at least 160 tiles of 256 rows x 256 tokens take the wide tiling (tokens loaded straight into LDS,
    the dequantization interleaved with the MFMAs, XCD-contiguous tile order): ragged rows, tokens (one token past a
    tile; 8 tokens into a third tile) and k (not a multiple of the 1024-input KT tile); sampled rows within the bound
    of fp64, the rows near every tile edge included."""
    L = make(8500 + bits + group, n, k, group, bits)
    x = gen_x(8600 + m, m * k).reshape(m, k)
    y = gemm(L, Dev.of(x), m)
    rows = np.unique(np.r_[0:96, 250:262, n // 2 - 40:n // 2 + 40, n - 300:n])
    w = dequant_host(L)
    assert within(y[:, rows], x, w[rows], k) <= 1.0


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_gemm_wide_tiles_exact_on_small_integer_operands(bits):
    """The wide tiling on small-integer operands and power-of-two scales: bit-exact against the fp64 product on every
    output (pins its operand layouts, the token DMA slots and the tile order), ldy stride padding untouched."""
    m, n, k, g = 300, 20600, 1024, 128
    L = make(8700 + bits, n, k, g, bits, scale_pow2=True)
    rng = np.random.default_rng(8701)
    x = f2bf_array(rng.integers(-3, 4, (m, k)).astype(np.float32))
    ld = n + 24
    y = gemm(L, Dev.of(x), m, ldy=ld, fill=0x7FC1)
    w = dequant_host(L)
    ref = bf2f_array(x).astype(np.float64) @ bf2f_array(w).astype(np.float64).T
    assert np.array_equal(y[:, :n], f2bf_array(ref.astype(np.float32)))
    assert (y[:, n:] == 0x7FC1).all()


def test_split_k_gemm_leaves_gemv_scratch_intact():
    """A narrow long-k GEMM splits k across workgroups (fp32 partials in the stream's scratch); the split-K GEMV
    launches on the same stream keep their row-range counters in the first 4 KB of that scratch, zero between
    launches: a 4-token down-shaped GEMV (5120 x 27648, split-K route) gives the same bits before and after it."""
    K = kernels()
    k = 27648
    D = make(8800, 5120, k, 128, 2)
    xg = gen_x(8801, 4 * k, 0.5)
    before = gemv(2, Dev.of(xg), 4, [D], k, 128)[0]
    check(K.ak_synchronize(), "sync")
    a = before.get(np.uint16, 4 * 5120)
    G = make(8802, 640, k, 128, 3)
    m = 256
    x = gen_x(8803, m * k).reshape(m, k)
    y = gemm(G, Dev.of(x), m)
    rows = np.r_[0:64, 576:640]
    assert within(y[:, rows], x, dequant_host(G)[rows], k) <= 1.0
    after = gemv(2, Dev.of(xg), 4, [D], k, 128)[0]
    check(K.ak_synchronize(), "sync")
    assert np.array_equal(after.get(np.uint16, 4 * 5120), a)


def test_graph_captured_before_scratch_growth_replays():
    """A split-K GEMV captured in a hipGraph addresses its stream's scratch; a later eager split-K GEMM on the same
    stream grows that scratch (a new buffer), and the replaced buffer stays allocated: replays after the growth, with
    new inputs each, equal eager launches."""
    from _lib import ptr_array, int_array
    K = kernels()
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    k, m = 27648, 4
    D = make(8900, 5120, k, 128, 2)
    X, Y = Dev(m * k * 2), Dev(m * 5120 * 2)
    G = make(8901, 640, k, 128, 3)
    mg = 256
    XG, YG = Dev.of(gen_x(8902, mg * k).reshape(mg, k)), Dev(mg * 640 * 2)
    stream, graph, exe = vp(), vp(), vp()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0

    def gemv_on(s, y):
        rc = K.ak_wq_gemv_kt_multi(2, X.p, m, 1, ptr_array([D.wt.p]), ptr_array([D.st.p]), ptr_array([y.p]),
                                   int_array([5120]), None, k, 128, 0, s)
        check(rc, "ak_wq_gemv_kt_multi")

    try:
        check(K.ak_memcpy_h2d(X.p, gen_x(8903, m * k, 0.5).ctypes.data, m * k * 2), "h2d")
        gemv_on(stream, Y)  # first split-K call on the stream: allocates its scratch
        assert hip.hipStreamSynchronize(stream) == 0
        assert hip.hipStreamBeginCapture(stream, ctypes.c_int(1)) == 0
        gemv_on(stream, Y)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        check(K.ak_wq_gemm_kt(3, XG.p, mg, G.wt.p, G.st.p, YG.p, 640, 0, k, 128, stream), "split-K GEMM")
        assert hip.hipStreamSynchronize(stream) == 0
        Ye = Dev(m * 5120 * 2)
        for rep in range(3):
            xh = gen_x(8910 + rep, m * k, 0.5)
            check(K.ak_memcpy_h2d(X.p, xh.ctypes.data, xh.nbytes), "h2d")
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            got = Y.get(np.uint16, m * 5120)
            gemv_on(stream, Ye)
            assert hip.hipStreamSynchronize(stream) == 0
            assert np.array_equal(got, Ye.get(np.uint16, m * 5120)), f"replay {rep}"
    finally:
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(stream)
