"""SiLU(gate) * up (ak_silu_mul / ak_silu_mul_part, reference kernels/src/fastmath/silu_mul.cu) on the GPU.

The reference's bits come from CUDA's fast-math exp and division, which are not restated here: parity is within one
bf16 unit in the last place of an fp64 evaluation of the same expression (numpy, test infrastructure), exact where the
value is exact (g = 0), and the share form bit-identical to the full form's columns with zeros elsewhere."""
import numpy as np
import pytest

from _lib import kernels, check, Dev, f2bf_array, bf2f_array

pytestmark = pytest.mark.gpu


def ref64(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


def within_one_ulp(got_bits, ref):
    got = bf2f_array(got_bits).astype(np.float64)
    a = np.abs(ref)
    ulp = np.where(a > 0, 2.0 ** (np.floor(np.log2(np.maximum(a, 1e-300))) - 7), 0.0)
    return np.abs(got - ref) <= ulp + 1e-38


def gate_up(rng, t, inter, scale=3.0):
    g = rng.standard_normal((t, inter)).astype(np.float32) * scale
    u = rng.standard_normal((t, inter)).astype(np.float32)
    g[0, :8] = [0.0, -0.0, 20.0, -20.0, 80.0, -80.0, 1e-3, -1e-3]
    gu = np.concatenate([g, u], axis=1)
    return f2bf_array(gu.ravel()).reshape(t, 2 * inter)


@pytest.mark.parametrize("t,inter", [(1, 27648), (5, 1024), (16, 8)])
def test_silu_mul_within_one_bf16_ulp(t, inter):
    rng = np.random.default_rng(t + inter)
    gu = gate_up(rng, t, inter)
    K = kernels()
    X, Y = Dev.of(gu), Dev(t * inter * 2)
    check(K.ak_silu_mul(X.p, Y.p, t, inter, None), "ak_silu_mul")
    check(K.ak_synchronize())
    got = Y.get(np.uint16, t * inter).reshape(t, inter)
    gf, uf = bf2f_array(gu[:, :inter]), bf2f_array(gu[:, inter:])
    ok = within_one_ulp(got, ref64(gf, uf))
    assert ok.all(), f"{int((~ok).sum())} of {ok.size} beyond one bf16 ulp"
    assert got[0, 0] == 0 or got[0, 0] == 0x8000  # g = 0


def test_silu_mul_part_equals_full_columns():
    rng = np.random.default_rng(3)
    inter, lo, npart = 512, 128, 256
    gu = gate_up(rng, 1, inter)
    K = kernels()
    X, Y = Dev.of(gu), Dev(inter * 2)
    check(K.ak_silu_mul(X.p, Y.p, 1, inter, None), "full")
    share = np.concatenate([gu[0, lo:lo + npart], gu[0, inter + lo:inter + lo + npart]])
    XS, YS = Dev.of(share), Dev.of(np.full(inter, 0x7FC1, dtype=np.uint16))
    check(K.ak_silu_mul_part(XS.p, YS.p, inter, lo, npart, None), "part")
    check(K.ak_synchronize())
    full, part = Y.get(np.uint16, inter), YS.get(np.uint16, inter)
    assert np.array_equal(part[lo:lo + npart], full[lo:lo + npart])
    assert np.all(part[:lo] == 0) and np.all(part[lo + npart:] == 0)
