"""Seeded ragged shapes through ak_wq_gemv_kt_multi, bit-exact against the oracle.

Forty-eight cases (each in both numerics) drawn from a fixed seed cover what the fixed-shape tests do not combine: rows not a multiple of 4
or 16 (padded row blocks), k a multiple of the group but not of 1024 (a padded last tile), 1..24 tokens (one launch,
8- and 16-token chunks), group 64 and 128, 2/3/4 bits, one to four segments of different sizes, and an ldy stride on
some segments.  Every output equals the oracle (the default numerics' exact group sums make every kernel shape give
the same bits); outputs past each segment's rows within the ldy stride stay untouched.
"""
import numpy as np
import pytest

from _lib import kernels, Dev, Linear, gemv, gen_container, gen_scales, gen_x, ora_fast, ora_exact

pytestmark = pytest.mark.gpu

LO = {4: -8, 3: -4, 2: -2}


def draw(i):
    rng = np.random.default_rng([20261202, i])
    bits = int(rng.choice([2, 3, 4]))
    group = int(rng.choice([64, 128]))
    k = group * int(rng.integers(1, 1 + 12288 // group))
    m = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24]))
    nseg = int(rng.integers(1, 5))
    ns = [int(rng.integers(1, 700)) for _ in range(nseg)]
    pad = [int(rng.integers(0, 9)) if rng.random() < 0.4 else 0 for _ in range(nseg)]
    return bits, group, k, m, ns, pad


CASES = [draw(i) for i in range(48)]


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


@pytest.mark.parametrize("mode", ["default", "exact"])
@pytest.mark.parametrize("i", range(len(CASES)))
def test_ragged_shape_matches_oracle(i, mode):
    """Default numerics against ora_gemv_fast_kt, the reference's exact fp32 order (ak_w4_set_mma(0)) against
    ora_gemv_exact_kt."""
    bits, group, k, m, ns, pad = CASES[i]
    print(f"case {i} ({mode}): bits {bits} group {group} k {k} m {m} n {ns} ldy pad {pad}", flush=True)
    K = kernels()
    K.ak_w4_set_mma(1 if mode == "default" else 0)
    lins = []
    for j, n in enumerate(ns):
        packed = gen_container(5000 + 10 * i + j, n, k, LO[bits], 1 << bits)
        scales = gen_scales(5500 + 10 * i + j, n * k // group)
        L = Linear(packed, scales, n, k, group, bits)
        assert L.rc == 0
        lins.append(L)
    ldy = [n + p for n, p in zip(ns, pad)]
    x = gen_x(6000 + i, m * k)
    X = Dev.of(x)
    sentinel = np.full(max(ldy) * m, 0x7FC1, dtype=np.uint16)  # a NaN pattern no output can take
    ys = [Dev.of(sentinel[: m * l].copy()) for l in ldy]
    gemv(bits, X, m, lins, k, group, ldy=ldy, ys=ys)
    for L, y, l in zip(lins, ys, ldy):
        got = y.get(np.uint16, m * l).reshape(m, l)
        wt, st = L.host_kt()
        want = (ora_fast if mode == "default" else ora_exact)(bits, x, m, wt, st, L.n, k, group)
        assert np.array_equal(got[:, :L.n], want), f"case {i}: segment of {L.n} rows differs"
        assert np.all(got[:, L.n:] == 0x7FC1), f"case {i}: writes past the segment's rows"
    K.ak_w4_set_mma(1)
