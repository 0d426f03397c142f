"""The MFMA route of ak_wq_gemv_kt_multi (csrc/wq_mm.hip): the default numerics above the measured crossover in m.

The route computes the integer numerics of the small-M kernels (x_int = trunc(x * 2^(148 - E)) per group, the exact
integer group sum rounded once to fp32, scale * 2^(E - 148), four group-slot accumulators per stripe, stripes added
left to right) with x_int fed to v_mfma_f32_16x16x32_f16 as two exact fp16 limbs, so every output must equal the
oracle's ora_gemv_fast_kt bit for bit -- the same bits a launch of fewer tokens on the integer kernels gives, which
is the reference's contract for batched rows (kernels/src/w4_gemv.cu:1075-1079).  Also checked: the reference's bound
|y - ref64| <= 1 bf16 ulp + 1e-6 * sum|x * w| (kernels/bench/test_w4.cu:123-141) against fp64, and the north-star
tolerance against ora_gemv_ref_f32 (reference.rs:53-71).  Size-independent properties at the benchmark shapes: a
token's outputs do not depend on the other tokens of the launch, on the segments launched with it, or on the token
count.
"""
import ctypes

import numpy as np
import pytest

from _lib import (kernels, Dev, Linear, gemv, gen_container, gen_scales, gen_x, ora_ref_f32, ora_ref_f64, ulp_bf16,
                  bf2f_array, check, ora_repack, ora_fast)

pytestmark = pytest.mark.gpu

G = 128


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    K.ak_w4_set_mma(1)
    K.ak_wq_set_mm_min(2)  # every launch of two or more tokens on the MFMA kernel
    yield K
    K.ak_w4_set_mma(-1)
    K.ak_wq_set_mm_min(-1)


def make_linear(seed, n, k, bits):
    packed = gen_container(seed, n, k, -(1 << (bits - 1)), 1 << bits)
    scales = gen_scales(seed + 1, n * k // G)
    return Linear(packed, scales, n, k, G, bits)


def rows_of(L, r0, r1):
    """The container and scales of rows [r0, r1) (row-major: k / 8 words and k / G scales per row)."""
    p = L.packed.reshape(L.n, L.k // 8)[r0:r1].ravel().copy()
    s = L.scales.reshape(L.n, L.k // G)[r0:r1].ravel().copy()
    return p, s


def check_rows(y, x, m, L, r0, r1, what=""):
    """y [m][n] (bf16 bits) rows r0..r1: bit-exact against the oracle's default numerics, and against fp64 (reference
    bound) and fp32."""
    p, s = rows_of(L, r0, r1)
    nr = r1 - r0
    rc, wt, st = ora_repack(L.bits, p, s, nr, L.k, G)
    assert rc == 0
    want = ora_fast(L.bits, x, m, wt, st, nr, L.k, G)
    got = np.ascontiguousarray(y[:, r0:r1])
    if not np.array_equal(got, want):
        bad = np.argwhere(got != want)[:4]
        raise AssertionError(f"{what} rows {r0}..{r1}: {int(np.sum(got != want))} outputs differ from the oracle, "
                             f"e.g. (token, row) {bad.tolist()}")
    ref64, mag = ora_ref_f64(x, m, p, s, nr, L.k, G)
    yy = y[:, r0:r1]
    err = np.abs(bf2f_array(yy).astype(np.float64) - ref64)
    bound = ulp_bf16(ref64) + 1e-6 * mag
    assert np.all(err <= bound), f"{what} rows {r0}..{r1}: worst {np.max(err / bound):.3f} of the bound"
    ref32 = ora_ref_f32(x, m, p, s, nr, L.k, G).astype(np.float64)
    # y is one of the two bf16 neighbours of a value within 2e-3 (relative, the measure of
    # bench_gemv.cu:146-148) of the fp32 reference
    y64 = bf2f_array(yy).astype(np.float64)
    rel = (np.abs(y64 - ref32) - ulp_bf16(ref32)) / (np.abs(ref32) + 1e-2)
    assert np.max(rel) <= 2e-3, f"{what}: {np.max(rel):.2e}"


def run(bits, x, m, lins, k, ldy=None):
    X = Dev.of(x)
    ys = gemv(bits, X, m, lins, k, G, ldy=ldy)
    return [y.get(np.uint16, m * (ldy[i] if ldy else L.n)).reshape(m, ldy[i] if ldy else L.n)
            for i, (y, L) in enumerate(zip(ys, lins))]


CASES = [  # bits, m, n, k: split-K (few rows per CU) and one-pass shapes, padded tiles and rows, 1..4 token tiles
    (2, 2, 512, 1024),
    (3, 5, 300, 2176),
    (4, 16, 1000, 5120),
    (3, 17, 256, 3072),
    (4, 40, 200, 1024),
    (2, 64, 128, 4096),
    (3, 128, 96, 2048),
    (2, 8, 320, 27648),
    (3, 4, 9000, 1024),
    (4, 9, 8500, 3072),
]


@pytest.mark.parametrize("bits,m,n,k", CASES)
def test_against_reference(bits, m, n, k):
    L = make_linear(1000 + bits * 7 + m, n, k, bits)
    x = gen_x(77 + m, m * k)
    (y,) = run(bits, x, m, [L], k)
    check_rows(y, x, m, L, 0, n, f"W{bits} m={m} {n}x{k}")


def test_chunked_activation_image():
    """16 tokens at k = 5120 on the one-pass route: the activation image (160 KB) is staged in two chunks."""
    L = make_linear(4242, 8800, 5120, 3)
    x = gen_x(4243, 16 * 5120)
    (y,) = run(3, x, 16, [L], 5120)
    for r0 in (0, 4352, 8800 - 160):
        check_rows(y, x, 16, L, r0, r0 + 160, "chunked")


def test_tokens_independent_of_launch():
    """A token's outputs are the same bits whatever tokens and segments share its launch (2, 16, 64, 100 tokens;
    q / k / v in one launch or each alone)."""
    k = 3072
    lins = [make_linear(500 + i, n, k, 4) for i, n in enumerate((640, 128, 128))]
    x = gen_x(501, 100 * k)
    full = run(4, x, 100, lins, k)
    for m in (2, 16, 64):
        part = run(4, x[: m * k], m, lins, k)
        for a, b in zip(part, full):
            assert np.array_equal(a, b[:m])
    for i, L in enumerate(lins):
        (alone,) = run(4, x[: 16 * k], 16, [L], k)
        assert np.array_equal(alone, full[i][:16])
    check_rows(full[0], x, 100, lins[0], 0, 640, "q segment")


def test_ldy_leaves_padding_untouched():
    k, n, m, ldy = 2048, 300, 6, 320
    L = make_linear(900, n, k, 2)
    x = gen_x(901, m * k)
    Y = Dev.of(np.full(m * ldy, 0x7FC1, dtype=np.uint16))
    gemv(2, Dev.of(x), m, [L], k, G, ldy=[ldy], ys=[Y])
    y = Y.get(np.uint16, m * ldy).reshape(m, ldy)
    assert np.all(y[:, n:] == 0x7FC1)
    check_rows(np.ascontiguousarray(y[:, :n]), x, m, L, 0, n, "ldy")


@pytest.mark.parametrize("m", [2, 4, 8, 16, 64])
def test_config3_qkv_and_o(m):
    """Config 3 at its benchmark shapes: QKV as q / k / v segments 5120 / 1024 / 1024 at k = 5120 and O 5120 x 5120,
    W4, sampled row windows (including each segment's last, padded block) against the reference."""
    k = 5120
    qkv = [make_linear(30 + i, n, k, 4) for i, n in enumerate((5120, 1024, 1024))]
    o = make_linear(40, 5120, k, 4)
    x = gen_x(41 + m, m * k)
    ys = run(4, x, m, qkv, k)
    for y, L in zip(ys, qkv):
        for r0 in (0, L.n - 64):
            check_rows(y, x, m, L, r0, r0 + 64, f"qkv m={m}")
    (yo,) = run(4, x, m, [o], k)
    for r0 in (0, 2560, 5120 - 64):
        check_rows(yo, x, m, o, r0, r0 + 64, f"o m={m}")


@pytest.mark.parametrize("bits,n,k,m", [(3, 55296, 5120, 4), (3, 55296, 5120, 16), (3, 55296, 5120, 128),
                                        (2, 5120, 27648, 16), (4, 152064, 5120, 16)])
def test_config4_shapes(bits, n, k, m):
    """Config 4's gate_up (also at 128 tokens), down and the W4 LM head on this route, sampled row windows."""
    L = make_linear(60 + bits, n, k, bits)
    x = gen_x(61 + m, m * k, 0.5 if k > 8192 else 1.0)
    (y,) = run(bits, x, m, [L], k)
    for r0 in (0, n // 2 - 37, n - 48):
        check_rows(y, x, m, L, r0, r0 + 48, f"W{bits} {n}x{k} m={m}")


def test_nonfinite_token_is_contained():
    """An Inf in one token's activations makes that token's outputs non-finite wherever the reference's fp32 path
    gives a non-finite output (here every output), and leaves the other tokens' outputs as they are."""
    k, n, m = 1024, 256, 4
    L = make_linear(70, n, k, 3)
    x = gen_x(71, m * k)
    (y0,) = run(3, x, m, [L], k)
    xi = x.copy()
    xi[2 * k + 5] = 0x7F80  # +Inf in token 2
    (y1,) = run(3, xi, m, [L], k)
    ref = ora_ref_f32(xi, m, L.packed, L.scales, n, k, G)[2]
    assert np.all(~np.isfinite(ref)) and np.all(~np.isfinite(bf2f_array(y1[2])))
    for t in (0, 1, 3):
        assert np.array_equal(y1[t], y0[t])


def test_fused_silu_down_on_this_route():
    """ak_wq_gemv_kt_silu (SiLU(gate) * up applied as the activations are staged) equals ak_silu_mul followed by the
    GEMV, bit for bit, at 4 and 16 tokens on this route."""
    K = kernels()
    inter, n = 3072, 512
    L = make_linear(80, n, inter, 2)
    for m in (4, 16):
        gu = gen_x(81 + m, m * 2 * inter, 2.0)
        X = Dev.of(gu)
        Yf = Dev(m * n * 2)
        check(K.ak_wq_gemv_kt_silu(2, X.p, m, L.wt.p, L.st.p, Yf.p, n, 0, inter, G, None), "ak_wq_gemv_kt_silu")
        A = Dev(m * inter * 2)
        check(K.ak_silu_mul(X.p, A.p, m, inter, None), "ak_silu_mul")
        (Ys,) = gemv(2, A, m, [L], inter, G)
        assert np.array_equal(Yf.get(np.uint16, m * n), Ys.get(np.uint16, m * n))
