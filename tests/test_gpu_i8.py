"""INT8 LM head GEMV (ak_i8_gemv, reference kernels/src/i8_gemv.cu:28-88) on the GPU: bit-identical to the oracle's
restatement of the reference's fp32 order (oracle/agq_oracle.c ora_i8_gemv), row j of an m-token call bit-identical to
the 1-token call, the row stride ldy, and the 152064 x 5120 LM head at m = 1."""
import numpy as np
import pytest

from _lib import kernels, check, Dev, f2bf_array, bf2f_array, oracle, ptr

pytestmark = pytest.mark.gpu


def data(seed, m, n, k):
    rng = np.random.default_rng(seed)
    x = f2bf_array(rng.standard_normal(m * k).astype(np.float32))
    q = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
    # per-row symmetric scale max|w| / 127 of a weight ~ N(0, 0.02)
    scale = (np.abs(rng.standard_normal(n)) * 0.02 / 127 * 3 + 1e-6).astype(np.float32)
    return x, q, scale


def ora(x, q, scale, m, n, k, ldy):
    y = np.zeros(m * ldy, dtype=np.uint16)
    oracle().ora_i8_gemv(ptr(x), ptr(q), ptr(scale), ptr(y), m, n, k, ldy)
    return y


def run(x, q, scale, m, n, k, ldy=None, fill=0x7FC1):
    K = kernels()
    ldy = ldy or n
    X, Q, S = Dev.of(x), Dev.of(q), Dev.of(scale)
    Y = Dev.of(np.full(m * ldy, fill, dtype=np.uint16))
    check(K.ak_i8_gemv(X.p, Q.p, S.p, Y.p, m, n, k, ldy, None), "ak_i8_gemv")
    check(K.ak_synchronize())
    return Y.get(np.uint16, m * ldy)


@pytest.mark.parametrize("m,n,k", [(1, 64, 5120), (1, 301, 1040), (1, 40, 16400), (3, 77, 16), (5, 130, 4096), (8, 19, 2064),
                                   (9, 40, 5120), (16, 33, 3072)])
def test_matches_oracle_bit_exact(m, n, k):
    x, q, scale = data(11 + m, m, n, k)
    got = run(x, q, scale, m, n, k)
    want = ora(x, q, scale, m, n, k, n)
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {got.size} outputs differ"


def test_order_known_answer_on_gpu():
    """The hand-computed order case of the oracle tests: the reference's order gives 2 (a left-to-right sum 1)."""
    k = 16 * 64
    xf = np.zeros(k, dtype=np.float32)
    xf[0], xf[16], xf[32], xf[48] = 2.0 ** 24, 1.0, -(2.0 ** 24), 1.0
    got = run(f2bf_array(xf), np.ones((1, k), dtype=np.int8), np.ones(1, dtype=np.float32), 1, 1, k)
    assert bf2f_array(got)[0] == 2.0


def test_rows_independent_of_m_and_ldy():
    m, n, k = 16, 150, 2048
    x, q, scale = data(3, m, n, k)
    ldy = n + 37
    full = run(x, q, scale, m, n, k, ldy=ldy).reshape(m, ldy)
    assert np.all(full[:, n:] == 0x7FC1), "columns past n were written"
    for j in (0, 5, 15):
        one = run(x[j * k:(j + 1) * k], q, scale, 1, n, k)
        assert np.array_equal(full[j, :n], one), f"token {j}"
    part = run(x[: 4 * k], q, scale, 4, n, k).reshape(4, n)
    assert np.array_equal(part, full[:4, :n])


def test_lm_head_shape():
    """152064 x 5120 at m = 1 (778 MB of int8 weights): bit-identical to the oracle."""
    m, n, k = 1, 152064, 5120
    x, q, scale = data(21, m, n, k)
    got = run(x, q, scale, m, n, k)
    want = ora(x, q, scale, m, n, k, n)
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {got.size} outputs differ"
