"""Non-finite and subnormal activations on the GPU, both numerics, every kernel family of the default numerics (the
line-load kernel at 1-2 tokens, the tokens-in-A-rows kernel at 3-16, split-K at long k, the any-m kernel at group 64).

Definition (include/agens_kernels.h, default numerics): a group holding a NaN adds NaN; a group holding an Inf (and
no NaN) adds S * scale * Inf with S the sum of sign(x) * q over its Inf inputs: +-Inf, or NaN where S = 0.  That is
the reference fp32 path's value (reference.rs:53-71: ga += x * q, acc += ga * s) wherever a group's Inf products
share one sign; these tests place one Inf per group, so every output must be NaN exactly where the fp32 path's is
and +-Inf with its sign.  Subnormal activations: the group sums stay exact, but the fp32 scale product
sc * 2^(E - 148) underflows for groups whose largest input is below about 2^-100 (it loses its precision at 2^-149),
so a token of subnormal inputs is checked bit for bit against the oracle and within an absolute 2^-100 of fp64
(outputs of such tokens are themselves below about 2^-110).  The exact numerics propagate like the reference's fp32 FMAs.
NaN payloads and signs are not compared (the CPU's and the GPU's default NaNs differ); NaN positions and every
other output bit are.
"""
import ctypes

import numpy as np
import pytest

from _lib import (kernels, check, Dev, Linear, gemv, gen_container, gen_scales, gen_x, ora_fast, ora_exact,
                  ora_ref_f32, ora_ref_f64, bf2f_array)

pytestmark = pytest.mark.gpu

PINF, NINF, QNAN, BIG = 0x7F80, 0xFF80, 0x7FC0, 0x7680  # BIG = 2^110


@pytest.fixture(scope="module", autouse=True)
def gpu():
    K = kernels()
    n = ctypes.c_int(0)
    assert K.ak_device_count(ctypes.byref(n)) == 0 and n.value >= 1, "no GPU visible"
    K.ak_w4_set_mma(1)
    K.ak_wq_set_mm_min(0)  # the integer-limb kernels at every m (the same numerics as the MFMA route)
    yield K
    K.ak_w4_set_mma(1)
    K.ak_w4_set_mma(-1)
    K.ak_wq_set_mm_min(-1)


def special_x(m, k, group, seed):
    """m tokens: token t % 4 == 0: one +Inf and one finite 2^110 in group 1 (x * 2^-107 would truncate to 8; the finite
    input must count 0); 1: a NaN in group 2; 2: -Inf in group 0 and +Inf in the last
    group; 3: every input subnormal (bf16 exponent field 0); the rest of each token N(0, 1)."""
    x = gen_x(seed, m * k).reshape(m, k)
    rng = np.random.default_rng(seed)
    for t in range(m):
        r = t % 4
        if r == 0:
            i = int(rng.integers(group))
            x[t, group + i] = PINF
            x[t, group + (i + 1 + int(rng.integers(group - 1))) % group] = BIG  # finite, counts 0 beside the Inf
        elif r == 1:
            x[t, 2 * group + int(rng.integers(group))] = QNAN
        elif r == 2:
            x[t, int(rng.integers(group))] = NINF
            x[t, k - group + int(rng.integers(group))] = PINF
        else:
            x[t] = (rng.integers(1, 128, k) | (rng.integers(0, 2, k) << 15)).astype(np.uint16)
    return x.reshape(-1)


def same_bits_nan_aware(got, want, what):
    gf, wf = bf2f_array(got), bf2f_array(want)
    gn, wn = np.isnan(gf), np.isnan(wf)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ ({int(np.sum(gn != wn))})"
    assert np.array_equal(got[~gn], want[~wn]), f"{what}: {int(np.sum(got[~gn] != want[~wn]))} outputs differ"


def classify_like_fp32(got, ref32, rows, what):
    """rows (token indices) whose only non-finite inputs are single Infs per group: NaN / +Inf / -Inf exactly where
    the reference's fp32 path has them."""
    g = bf2f_array(got)
    for t in rows:
        a, b = g[t], ref32[t]
        assert np.array_equal(np.isnan(a), np.isnan(b)), f"{what}: token {t}: NaN positions"
        assert np.array_equal(np.isposinf(a), np.isposinf(b)), f"{what}: token {t}: +Inf positions"
        assert np.array_equal(np.isneginf(a), np.isneginf(b)), f"{what}: token {t}: -Inf positions"


CASES = [(4, 128, 256, 5120, 1), (3, 128, 256, 5120, 2), (2, 128, 300, 5120, 4), (4, 128, 300, 5120, 8),
         (3, 128, 256, 5120, 16), (2, 128, 512, 27648, 1), (3, 128, 512, 27648, 4), (4, 128, 256, 27648, 16),
         (3, 64, 256, 3072, 4), (4, 64, 96, 3072, 1)]


@pytest.mark.parametrize("bits,group,n,k,m", CASES)
def test_nonfinite_and_subnormal_activations(bits, group, n, k, m):
    K = kernels()
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed = gen_container(7000 + bits, n, k, lo, span)
    scales = gen_scales(7001 + bits, n * k // group)
    L = Linear(packed, scales, n, k, group, bits)
    check(L.rc)
    wt, st = L.host_kt()
    x = special_x(m, k, group, 7100 + m)
    X = Dev.of(x)
    ref32 = ora_ref_f32(x, m, packed, scales, n, k, group)
    ref64, mag = ora_ref_f64(x, m, packed, scales, n, k, group)
    single = [t for t in range(m) if t % 4 in (0, 2)]
    for mode, ora in ((1, ora_fast), (0, ora_exact)):
        K.ak_w4_set_mma(mode)
        try:
            (Y,) = gemv(bits, X, m, [L], k, group)
        finally:
            K.ak_w4_set_mma(1)
        y = Y.get(np.uint16, m * n).reshape(m, n)
        what = f"{'default' if mode else 'exact'} bits={bits} g={group} n={n} k={k} m={m}"
        same_bits_nan_aware(y, ora(bits, x, m, wt, st, n, k, group), what)
        classify_like_fp32(y, ref32, single, what)
        for t in range(m):
            if t % 4 == 1:
                assert np.all(np.isnan(bf2f_array(y[t]))), f"{what}: a NaN input leaves every output NaN"
            if t % 4 == 3:
                err = np.abs(bf2f_array(y[t]).astype(np.float64) - ref64[t])
                assert np.all(err <= 2.0 ** -100), f"{what}: subnormal token {t}: {err.max()}"


@pytest.mark.parametrize("bits,n,k,m", [(3, 256, 5120, 16), (2, 300, 5120, 24), (4, 256, 3072, 40),
                                        (3, 512, 27648, 17)])
def test_nonfinite_on_the_mfma_route(bits, n, k, m):
    """The fp16-MFMA route (forced from 2 tokens) on the same non-finite and subnormal activations: the oracle's bits
    (NaN positions, every other output bit), as the integer kernels give them."""
    K = kernels()
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed = gen_container(7200 + bits, n, k, lo, span)
    scales = gen_scales(7201 + bits, n * k // 128)
    L = Linear(packed, scales, n, k, 128, bits)
    check(L.rc)
    wt, st = L.host_kt()
    x = special_x(m, k, 128, 7300 + m)
    X = Dev.of(x)
    ys = {}
    for mmin in (2, 0):
        K.ak_wq_set_mm_min(mmin)
        try:
            (Y,) = gemv(bits, X, m, [L], k, 128)
        finally:
            K.ak_wq_set_mm_min(0)
        ys[mmin] = Y.get(np.uint16, m * n).reshape(m, n)
    what = f"MFMA route bits={bits} n={n} k={k} m={m}"
    same_bits_nan_aware(ys[2], ora_fast(bits, x, m, wt, st, n, k, 128), what)
    same_bits_nan_aware(ys[2], ys[0], what + " vs the integer kernels")
