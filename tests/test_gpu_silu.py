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


# ------------------------------------------------------------------------------------------------ fused into the GEMV
from _lib import gen_container, gen_scales, Linear, gemv, wq_step, Chain  # noqa: E402


def down_linear(seed, bits, n, inter, group=128):
    lo, span = -(1 << (bits - 1)), 1 << bits
    L = Linear(gen_container(seed, n, inter, lo, span), gen_scales(seed + 1, n * inter // group), n, inter, group,
               bits)
    check(L.rc, "repack")
    return L


def fused_and_separate(L, gu, m, inter):
    K = kernels()
    X = Dev.of(gu)
    Yf = Dev.of(np.full(m * L.n, 0x7FC1, dtype=np.uint16))
    rc = K.ak_wq_gemv_kt_silu(L.bits, X.p, m, L.wt.p, L.st.p, Yf.p, L.n, 0, inter, L.group, None)
    check(rc, "ak_wq_gemv_kt_silu")
    A = Dev(m * inter * 2)
    check(K.ak_silu_mul(X.p, A.p, m, inter, None), "ak_silu_mul")
    (Ys,) = gemv(L.bits, A, m, [L], inter, L.group)
    check(K.ak_synchronize())
    return Yf.get(np.uint16, m * L.n), Ys.get(np.uint16, m * L.n)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("m", [1, 2, 4, 9, 16])
def test_fused_down_equals_silu_then_gemv(bits, m):
    """The down projection of a 32B layer (5120 x 27648: split-K launches at every m), fused against the two calls."""
    n, inter = 5120, 27648
    L = down_linear(300 + bits, bits, n, inter)
    gu = gate_up(np.random.default_rng(m + 10 * bits), m, inter, scale=2.0)
    fused, sep = fused_and_separate(L, gu, m, inter)
    assert np.array_equal(fused, sep), f"{int(np.sum(fused != sep))} of {fused.size} differ"


@pytest.mark.parametrize("m,n,inter", [(1, 300, 2560), (3, 77, 1152), (8, 130, 4096)])
def test_fused_small_shapes(m, n, inter):
    L = down_linear(77, 3, n, inter)
    gu = gate_up(np.random.default_rng(n), m, inter)
    fused, sep = fused_and_separate(L, gu, m, inter)
    assert np.array_equal(fused, sep)


def test_fused_group64_is_invalid():
    K = kernels()
    L = down_linear(5, 4, 64, 1024, group=64)
    X, Y = Dev(2 * 1024 * 2), Dev(64 * 2)
    assert K.ak_wq_gemv_kt_silu(4, X.p, 1, L.wt.p, L.st.p, Y.p, 64, 0, 1024, 64, None) == 1


@pytest.mark.parametrize("m", [1, 2])
def test_chain_with_fused_down(m):
    """gate_up -> down(SiLU(gate) * up) for two 32B layers in one chained launch, against separate calls."""
    K = kernels()
    H, INTER = 5120, 27648
    x = Dev.of(f2bf_array(np.random.default_rng(4).standard_normal(m * H).astype(np.float32)))
    steps, flow = [], []
    xin = x
    for li, bits in enumerate((3, 2)):
        lo, span = -(1 << (bits - 1)), 1 << bits
        gu = Linear(gen_container(500 + li, 2 * INTER, H, lo, span),
                    gen_scales(501 + li, 2 * INTER * H // 128, 1.0 / np.sqrt(H * 5.5)), 2 * INTER, H, 128, bits)
        dn = down_linear(600 + li, bits, H, INTER)
        ygu, yh = Dev(m * 2 * INTER * 2), Dev(m * H * 2)
        steps += [wq_step(bits, xin, m, [gu], [ygu], H), wq_step(bits, ygu, m, [dn], [yh], INTER, act=1)]
        flow += [(gu, xin, ygu, H, 0), (dn, ygu, yh, INTER, 1)]
        xin = yh
    ch = Chain(steps)
    assert ch.chained
    ch.run()
    check(K.ak_synchronize())
    assert K.ak_wq_chain_status() == 0
    got = [y.get(np.uint16, m * L.n) for L, _, y, _, _ in flow]
    for L, xi, y, k, act in flow:  # the same steps as separate calls, in order
        if act:
            A = Dev(m * k * 2)
            check(K.ak_silu_mul(xi.p, A.p, m, k, None), "silu")
            gemv(L.bits, A, m, [L], k, 128, ys=[y])
        else:
            gemv(L.bits, xi, m, [L], k, 128, ys=[y])
    check(K.ak_synchronize())
    for i, (L, _, y, _, _) in enumerate(flow):
        assert np.array_equal(got[i], y.get(np.uint16, m * L.n)), f"step {i}"
