"""Batch-invariant bf16 GEMV (ak_bf16_gemv_bi / _ld, reference kernels/src/bi_gemv.cu:270-356) on the GPU.

The reference's bits come from its tensor-core MMA's internal accumulation, which no other hardware reproduces, so
parity is: bit-exact where every partial sum is an exact fp32 integer (small-integer operands: any summation order
gives the exact value, which pins the operand and output layout), within fp32-accumulation tolerance of an fp64 product
elsewhere (numpy, test infrastructure), and the reference's contract that row t of an m-token call is bit-identical to
the 1-token call, for every m up to 128."""
import numpy as np
import pytest

from _lib import kernels, check, Dev, f2bf_array, bf2f_array

pytestmark = pytest.mark.gpu


def run(x, w, bias, m, n, k, ldy=None, fill=0x7FC1):
    K = kernels()
    X, W = Dev.of(x), Dev.of(w)
    B = Dev.of(bias) if bias is not None else None
    ld = ldy or n
    Y = Dev.of(np.full(m * ld, fill, dtype=np.uint16))
    if ldy is None:
        rc = K.ak_bf16_gemv_bi(X.p, W.p, B.p if B else None, Y.p, m, n, k, None)
    else:
        rc = K.ak_bf16_gemv_bi_ld(X.p, W.p, B.p if B else None, Y.p, m, n, k, ldy, None)
    check(rc, "ak_bf16_gemv_bi")
    check(K.ak_synchronize())
    return Y.get(np.uint16, m * ld)


@pytest.mark.parametrize("m,n,k", [(1, 24, 4096), (5, 48, 96), (16, 100, 4096), (17, 33, 2048), (40, 16, 32),
                                   (128, 70, 1024)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_exact_integer_operands(m, n, k, with_bias):
    rng = np.random.default_rng(m * 1000 + n + k)
    xi = rng.integers(-4, 5, size=(m, k))
    wi = rng.integers(-8, 9, size=(n, k))
    bi = rng.integers(-64, 65, size=n) if with_bias else None
    S = xi.astype(np.int64) @ wi.astype(np.int64).T + (bi[None, :] if with_bias else 0)
    got = run(f2bf_array(xi.astype(np.float32).ravel()), f2bf_array(wi.astype(np.float32).ravel()),
              f2bf_array(bi.astype(np.float32)) if with_bias else None, m, n, k).reshape(m, n)
    want = f2bf_array(S.astype(np.float32).ravel()).reshape(m, n)
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {got.size} differ"


@pytest.mark.parametrize("m,n,k", [(1, 24, 5120), (8, 48, 7168), (33, 200, 3072)])
def test_within_fp32_accumulation_tolerance(m, n, k):
    rng = np.random.default_rng(n + k)
    x = f2bf_array(rng.standard_normal(m * k).astype(np.float32))
    w = f2bf_array((rng.standard_normal(n * k) * 0.02).astype(np.float32))
    b = f2bf_array((rng.standard_normal(n) * 0.1).astype(np.float32))
    y = bf2f_array(run(x, w, b, m, n, k)).reshape(m, n).astype(np.float64)
    xf = bf2f_array(x).reshape(m, k).astype(np.float64)
    wf = bf2f_array(w).reshape(n, k).astype(np.float64)
    ref = xf @ wf.T + bf2f_array(b).astype(np.float64)[None, :]
    mag = np.abs(xf) @ np.abs(wf).T + np.abs(bf2f_array(b)).astype(np.float64)[None, :]
    # one bf16 rounding (2^-9 relative, with a margin) plus fp32 summation error (k 2^-24 of sum |x w|)
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + mag * k * 2.0 ** -24)


def test_rows_bit_identical_for_every_m_and_ldy():
    n, k = 72, 3072
    rng = np.random.default_rng(9)
    x = f2bf_array(rng.standard_normal(128 * k).astype(np.float32))
    w = f2bf_array((rng.standard_normal(n * k) * 0.02).astype(np.float32))
    b = f2bf_array((rng.standard_normal(n) * 0.1).astype(np.float32))
    full = run(x, w, b, 128, n, k, ldy=n + 9).reshape(128, n + 9)
    assert np.all(full[:, n:] == 0x7FC1), "columns past n were written"
    for m in (1, 3, 16, 17, 50):
        part = run(x[: m * k], w, b, m, n, k).reshape(m, n)
        assert np.array_equal(part, full[:m, :n]), f"m = {m}"
    one = run(x[77 * k: 78 * k], w, b, 1, n, k)
    assert np.array_equal(one, full[77, :n])
